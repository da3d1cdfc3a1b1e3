"""RecoverSSM verify / grouped commit for Gated DeltaNet on AMD Instinct MI355X.

Drop-in for the hot path of the reference plugin ``gdn_recoverssm_ascend``:
the same module names (``kernels``, ``grouped_commit``) and public API, backed
by hand-written gfx950 HIP kernels behind the C ABI of
``include/gdn_recoverssm_hip.h``. Importing the package does not touch the GPU;
the HIP library is loaded on first launch and its absence is an error.
"""

from .grouped_commit import (  # noqa: F401
    CommitEntry,
    GroupedCommitBucket,
    GroupedCommitCoordinator,
    prepare_grouped_commit,
)
from .kernels import (  # noqa: F401
    MAX_SPEC_QUERY_LEN,
    NULL_BLOCK_ID,
    GDNRecoverSSMCommitContext,
    PendingCommit,
    ReplayRecordBuffers,
    continue_pending,
    counts,
    gdn_recoverssm_verify,
    gdn_recoverssm_verify_deferred,
    gdn_recoverssm_verify_gated,
    record_geometry_bytes,
    record_nbytes,
)


def initialize():
    """Load the HIP library and check its ABI version (raises if absent)."""
    from . import _native

    return _native.load()


__all__ = [
    "CommitEntry",
    "GDNRecoverSSMCommitContext",
    "GroupedCommitBucket",
    "GroupedCommitCoordinator",
    "MAX_SPEC_QUERY_LEN",
    "NULL_BLOCK_ID",
    "PendingCommit",
    "ReplayRecordBuffers",
    "continue_pending",
    "counts",
    "gdn_recoverssm_verify",
    "gdn_recoverssm_verify_deferred",
    "gdn_recoverssm_verify_gated",
    "initialize",
    "prepare_grouped_commit",
    "record_geometry_bytes",
    "record_nbytes",
]
