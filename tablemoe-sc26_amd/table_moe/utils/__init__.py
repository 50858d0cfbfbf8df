from .modality import ModalityContext

__all__ = ["ModalityContext"]
