from .qwen2 import Qwen2, Qwen2Meta

__all__ = ["Qwen2", "Qwen2Meta"]
