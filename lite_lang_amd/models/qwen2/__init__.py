from .model import Qwen2Model, Qwen2ModelRunner  # noqa: F401
from .weights import Qwen2Config  # noqa: F401
