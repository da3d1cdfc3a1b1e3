"""Ahead-of-time build of the gfx950 HIP library (``libgdn_recoverssm_hip.so``).

``python -m gdn_recoverssm_ascend._build`` (or ``build()``) compiles every
``csrc/*.hip`` source with hipcc for gfx950 into one shared library placed next
to this package (``_lib/``), where the ctypes loader finds it. The build is
in-tree so the artefact travels with the source tree; nothing is JIT-compiled
at run time.
"""

from __future__ import annotations

import hashlib
import os
import shutil
import subprocess
import sys
import tempfile

PKG_DIR = os.path.dirname(os.path.abspath(__file__))
PROJECT_DIR = os.path.dirname(PKG_DIR)
REPO_DIR = os.path.dirname(PROJECT_DIR)
CSRC_DIR = os.path.join(PROJECT_DIR, "csrc")
INCLUDE_DIR = os.path.join(REPO_DIR, "include")
LIB_DIR = os.path.join(PKG_DIR, "_lib")
LIB_NAME = "libgdn_recoverssm_hip.so"
LIB_PATH = os.path.join(LIB_DIR, LIB_NAME)
# The source digest of a built library, written beside it by build().
DIGEST_SUFFIX = ".digest"
# Synthetic traffic probes for bench.py's measured ceilings (not part of the
# verify / commit path): a library of their own, built by build_probe(), a
# step apart from the product library's build().
PROBE_SRC = os.path.join(CSRC_DIR, "probe", "traffic_probe.hip")
PROBE_LIB_PATH = os.path.join(LIB_DIR, "libgdn_recoverssm_probe.so")
ARCH = os.environ.get("GDN_OFFLOAD_ARCH", "gfx950")


def sources() -> list[str]:
    return sorted(os.path.join(CSRC_DIR, f) for f in os.listdir(CSRC_DIR) if f.endswith(".hip"))


def source_digest() -> str:
    """SHA-1 over the kernel sources and the C header: identifies the code a
    profile was taken of."""
    h = hashlib.sha1()
    files = sorted(f for f in os.listdir(CSRC_DIR) if f.endswith((".hip", ".cuh")))
    for path in [os.path.join(CSRC_DIR, f) for f in files] + [os.path.join(INCLUDE_DIR, "gdn_recoverssm_hip.h")]:
        h.update(os.path.basename(path).encode())
        with open(path, "rb") as f:
            h.update(f.read())
    return h.hexdigest()


def hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), shutil.which("hipcc"), "/opt/rocm/bin/hipcc"):
        if cand and os.path.exists(cand):
            return cand
    raise RuntimeError("hipcc not found: the gfx950 HIP library cannot be built")


def compile_flags() -> list[str]:
    return [
        f"--offload-arch={ARCH}",
        "-O3",
        "-std=c++17",
        "-fPIC",
        "-Wall",
        "-Wno-unused-function",
        # Packed FP32 instructions stay off: plain FP32 VALU code only.
        "-Xclang",
        "-target-feature",
        "-Xclang",
        "-packed-fp32-ops",
        f"-I{INCLUDE_DIR}",
        f"-I{CSRC_DIR}",
    ]


def _compile(cc: str, src: str, obj: str, verbose: bool):
    cmd = [cc, *compile_flags(), "-c", src, "-o", obj]
    if verbose:
        print(" ".join(cmd), flush=True)
    r = subprocess.run(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT)
    text = r.stdout.decode(errors="replace")
    text = "\n".join(l for l in text.splitlines() if "packed-fp32-ops" not in l and l.strip() != "1 warning generated.")
    return src, obj, r.returncode, text


def build(verbose: bool = False, jobs: int = min(8, os.cpu_count() or 1)) -> str:
    """Compile every library source (in parallel, largest first), link the
    shared library and record the digest of the sources it was built from
    beside it."""
    from concurrent.futures import ThreadPoolExecutor

    digest = source_digest()
    os.makedirs(LIB_DIR, exist_ok=True)
    cc = hipcc()
    srcs = sorted(sources(), key=os.path.getsize, reverse=True)
    srcs = sorted(srcs, key=lambda p: 0 if os.path.basename(p).startswith("verify_") else 1)
    with tempfile.TemporaryDirectory(prefix="gdn_build_") as tmp:

        def compile_one(src):
            return _compile(cc, src, os.path.join(tmp, os.path.basename(src) + ".o"), verbose)

        with ThreadPoolExecutor(max_workers=max(1, jobs)) as pool:
            results = list(pool.map(compile_one, srcs))
        errors = [f"{src}:\n{text}" for src, _, rc, text in results if rc != 0]
        if verbose:
            for src, _, rc, text in results:
                if rc == 0 and text.strip():
                    print(text)
        if errors:
            raise RuntimeError("hipcc failed:\n" + "\n".join(errors))
        objs = [obj for _, obj, _, _ in results]
        tmp_lib = LIB_PATH + ".tmp"
        link = [cc, f"--offload-arch={ARCH}", "-shared", "-fPIC", *objs, "-o", tmp_lib]
        r = subprocess.run(link, stdout=subprocess.PIPE, stderr=subprocess.STDOUT)
        if r.returncode != 0:
            raise RuntimeError("hipcc link failed:\n" + r.stdout.decode(errors="replace"))
        os.replace(tmp_lib, LIB_PATH)
    with open(LIB_PATH + DIGEST_SUFFIX, "w") as f:
        f.write(digest + "\n")
    return LIB_PATH


def build_probe(verbose: bool = False) -> str:
    """The traffic probes bench.py times beside the kernels (synthetic
    kernels moving each kernel's bytes in its access pattern): a library of
    their own, which the verify / commit library does not need."""
    os.makedirs(LIB_DIR, exist_ok=True)
    cc = hipcc()
    with tempfile.TemporaryDirectory(prefix="gdn_probe_") as tmp:
        src, obj, rc, text = _compile(cc, PROBE_SRC, os.path.join(tmp, "traffic_probe.o"), verbose)
        if rc != 0:
            raise RuntimeError(f"hipcc failed:\n{src}:\n{text}")
        r = subprocess.run([cc, f"--offload-arch={ARCH}", "-shared", "-fPIC", obj, "-o", PROBE_LIB_PATH + ".tmp"],
                           stdout=subprocess.PIPE, stderr=subprocess.STDOUT)
        if r.returncode != 0:
            raise RuntimeError("hipcc link failed:\n" + r.stdout.decode(errors="replace"))
        os.replace(PROBE_LIB_PATH + ".tmp", PROBE_LIB_PATH)
    return PROBE_LIB_PATH


def built_digest(path: str) -> str | None:
    """The source digest recorded beside a built library (None when absent)."""
    try:
        with open(path + DIGEST_SUFFIX) as f:
            return f.read().strip()
    except OSError:
        return None


if __name__ == "__main__":
    print(build(verbose="-v" in sys.argv))
    print(build_probe(verbose="-v" in sys.argv))
