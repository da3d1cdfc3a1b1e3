"""RecoverSSM verify / grouped commit for Gated DeltaNet on AMD Instinct MI355X.

Drop-in for the hot path of the reference plugin ``gdn_recoverssm_ascend``:
the same module names (``kernels``, ``grouped_commit``) and public API, backed
by hand-written gfx950 HIP kernels behind the C ABI of
``include/gdn_recoverssm_hip.h``. Importing the package does not touch the GPU;
the HIP library is loaded on first launch and its absence is an error.
"""

from .grouped_commit import (  # noqa: F401
    CommitEntry,
    DeferredGroupedCommit,
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


def set_state_cache_retain(nbytes: int) -> int:
    """Cache hint of this implementation (the reference has none): how many
    bytes of checkpoint state each verify launch (``gdn_recoverssm_verify``,
    ``gdn_recoverssm_verify_gated``) reads with ordinary loads, counted from
    the end of its batch; earlier rows read their pages non-temporally. This
    is the process-wide setting, used by every call that does not pass its
    own ``state_cache_retain``. The default, 64 MiB, suits the model's decode
    step, where other layers' verifies run before any commit re-reads a
    layer's pages (B=128 layers ran fastest with it). A caller whose commit
    directly follows the verify of the same pages (one layer's verify,
    sampling, commit) gains from 256 MiB, the MI355X memory-side cache: the
    commit then finds the last-read pages there. The deferred verify reads
    every row non-temporally whatever the setting. Results are identical
    either way. Returns the previous value."""
    from . import _native

    if int(nbytes) < 0:
        raise ValueError("GDN RecoverSSM: the retained state bytes must be >= 0")
    return int(_native.load().gdn_recoverssm_set_state_cache_retain(int(nbytes)))


__all__ = [
    "CommitEntry",
    "DeferredGroupedCommit",
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
    "set_state_cache_retain",
]
