from .qwen_topk_softmax import qwen_topk_softmax

__all__ = ["qwen_topk_softmax"]
