from .importance import cache_last_token_attention, compute_and_cache_importance, last_query_importance
from .modality import ModalityContext

__all__ = ["ModalityContext", "compute_and_cache_importance", "cache_last_token_attention", "last_query_importance"]
