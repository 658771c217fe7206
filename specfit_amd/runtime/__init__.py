"""Drop-in runtime of the offloaded Qwen3-MoE verification path
(mirrors the public names of the reference's ``specfit.runtime``)."""
from .cache_observer import (CacheTransition, CacheTransitionCounters, CacheTransitionObserver,
                             RecordingCacheTransitionObserver,
                             aggregate_cache_transition_counters)
from .cache_snapshot import CacheSlotSnapshot, GpuExpertCacheSnapshot, PendingTransferSnapshot
from .gpu_expert_cache import GpuExpertCache
from .lease import ExpertCacheStats, ExpertLease, NoEvictableSlotError
from .qwen3_offloaded_experts import (ExpertExecutionPolicy, Qwen3OffloadedExperts,
                                      ReductionMode)
from .qwen3_expert_prefetch import Qwen3ExpertPrefetch
from .qwen3_offloaded_model import (LoadedOffloadedQwen3, PackedExpertBackingMode,
                                    Qwen3LoadTimings, build_offloaded_qwen3, load_offloaded_qwen3)
from .qwen3_attention import Qwen3AttentionHip, install_hip_attention
from .qwen3_norm import Qwen3RMSNormHip, install_hip_norms
from .qwen3_router import Qwen3MoeTopKRouterHip
from .replay import (ExpertAccessReplayResult, LogicalReplayError, LogicalReplayEvent,
                     ReplayCounters, ReplaySlotState, replay_qwen3_access_cycles,
                     replay_qwen3_accesses)
from .state import ExpertKey
from .trace import RuntimeEventKind
from .tree_attention import TREE_ATTENTION, register_tree_attention, tree_attention_forward
from .tree_verify import (Eagle3DraftTree, TreeVerification, compact_tree_cache, synthetic_tree,
                          verify_draft_tree)

__all__ = [
    "CacheSlotSnapshot", "CacheTransition", "CacheTransitionCounters",
    "CacheTransitionObserver", "ExpertCacheStats", "ExpertExecutionPolicy", "ExpertKey",
    "ExpertLease", "GpuExpertCache", "GpuExpertCacheSnapshot", "NoEvictableSlotError",
    "LoadedOffloadedQwen3", "PackedExpertBackingMode", "PendingTransferSnapshot", "Qwen3ExpertPrefetch", "Qwen3LoadTimings",
    "Qwen3MoeTopKRouterHip", "Qwen3OffloadedExperts", "Qwen3RMSNormHip", "build_offloaded_qwen3",
    "install_hip_norms", "Qwen3AttentionHip", "install_hip_attention",
    "load_offloaded_qwen3",
    "RecordingCacheTransitionObserver", "ReductionMode", "RuntimeEventKind",
    "aggregate_cache_transition_counters",
    "ExpertAccessReplayResult", "LogicalReplayError", "LogicalReplayEvent", "ReplayCounters",
    "ReplaySlotState", "replay_qwen3_access_cycles", "replay_qwen3_accesses",
    "Eagle3DraftTree", "TREE_ATTENTION", "TreeVerification", "compact_tree_cache",
    "register_tree_attention", "synthetic_tree", "tree_attention_forward", "verify_draft_tree",
]
