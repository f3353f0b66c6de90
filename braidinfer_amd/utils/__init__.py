"""Host utilities under the module names of braidinfer/utils."""
from .loader import default_weight_loader, load_model

__all__ = ["default_weight_loader", "load_model"]
