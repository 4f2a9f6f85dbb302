"""minispeed_amd — minispeed's gradient-accumulation boundary step on MI355X.

Same public surface as ``import minispeed as ms`` (minispeed/__init__.py:23-46)
for the training-step path: ``initialize``, ``DeepSpeedEngine``,
``DeepSpeedConfig``, ``ConfigError``, ``ZeROOptimizer``, ``DynamicLossScaler``,
``WarmupLR``, ``WarmupDecayLR``, ``Timers``, ``set_seed`` and ``comm``.  The
boundary step (flatten, inf/nan check, unscale, global norm, clip, AdamW,
master->model cast) runs as hand-written gfx950 HIP kernels from
``libminispeed_boundary.so``.
"""

from . import comm
from .config import ConfigError, DeepSpeedConfig
from .engine import DeepSpeedEngine, initialize
from .optim import WarmupDecayLR, WarmupLR
from .precision import DynamicLossScaler
from .utils import Timers, set_seed
from .zero import ZeROOptimizer

__version__ = "0.1.0"

__all__ = [
    "initialize",
    "DeepSpeedEngine",
    "DeepSpeedConfig",
    "ConfigError",
    "ZeROOptimizer",
    "DynamicLossScaler",
    "WarmupLR",
    "WarmupDecayLR",
    "Timers",
    "set_seed",
    "comm",
    "__version__",
]
