from .fp16_fused_expert import expert_swiglu, maybe_run_fp16_fused_expert
from .grouped_expert import GroupedExperts, SharedExperts
from .qwen_topk_softmax import qwen_topk_softmax

__all__ = ["maybe_run_fp16_fused_expert", "qwen_topk_softmax", "expert_swiglu", "GroupedExperts", "SharedExperts"]
