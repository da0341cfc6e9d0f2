"""Dispatcher-Hybrid for MI355X: the attention-light causal LM whose dyadic shift-and-sum mixer
runs on hand-written gfx950 HIP kernels (parallel gate pipeline + level scan, one-kernel decode
step) behind the reference package's public API.
"""

from .configuration_dispatcher import DispatcherConfig
from .modeling_dispatcher import DispatcherHybridForCausalLM

__version__ = "0.1.2"
__all__ = ["DispatcherConfig", "DispatcherHybridForCausalLM"]

try:  # let AutoConfig / AutoModelForCausalLM resolve the architecture
    from transformers import AutoConfig, AutoModelForCausalLM

    AutoConfig.register("dispatcher-hybrid", DispatcherConfig)
    AutoModelForCausalLM.register(DispatcherConfig, DispatcherHybridForCausalLM)
except Exception:  # pragma: no cover - already registered
    pass
