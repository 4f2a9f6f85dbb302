"""DeepSpeed-style JSON config, the subset minispeed accepts.

Same keys, defaults and validation errors as minispeed/config.py:53-202 so a
minispeed config drives this package unchanged:

    train_batch_size / train_micro_batch_size_per_gpu /
    gradient_accumulation_steps                        (config.py:61-83)
    dtype | fp16.enabled | bf16.enabled                (config.py:86, 163-176)
    fp16.{loss_scale, initial_scale_power, loss_scale_window}  (config.py:88-98)
    gradient_clipping                                  (config.py:101-102)
    zero_optimization.stage (+ rejected offload keys)  (config.py:105-123)
    optimizer.{type, params}                           (config.py:126-139)
    scheduler.{type, params}                           (config.py:142-155)
    steps_per_print, seed, drop_overflow_on_loss       (config.py:158-160)

One section is specific to this package and ignored by minispeed:

    "hip_boundary": {"materialize_flat_grad": false, "contiguous_gradients": false,
                     "state_spacing_gib": "auto", "stage3_gather_reuse": false}

With ``materialize_flat_grad`` the ragged-grad kernel also writes the fp32
flat gradient buffer and the AdamW kernel reads it back (36 B/param for half
grads); by default the AdamW kernel re-reads the ragged half gradients and
the flat buffer is never written (30 B/param).  Both give identical results.

``contiguous_gradients`` (opt-in) accumulates every micro-batch gradient in
fp32 straight into a flat buffer as backward produces it, instead of in the
parameter dtype in ``param.grad``; ``param.grad`` is released after each
backward.  This changes the numerics (fp32 instead of half accumulation), so
it is not bitwise minispeed and is off by default.

``state_spacing_gib`` places the fp32 masters, exp_avg and exp_avg_sq of all
groups: with a number of GiB they lie in one allocation (the state arena) of
three windows of that size, array j at the start of window j; 0 gives three
separate allocations; "auto" (the default) uses 36 GiB windows for states of
256 MiB to 36 GiB per array when the 108 GiB arena takes at most half of
the free device memory, and separate allocations otherwise.  On MI355X the
fused AdamW kernel streams the three arrays 5-15% faster when they lie far
apart in physical memory (1.3B params: 5.64-5.74 against 6.1-6.9 ms for
separate allocations; 124M params: 0.52 against 0.61-0.63 ms).  The arena is
carved through torch's caching allocator: the state holds only its own
bytes, and the rest of the arena goes back to the allocator as free blocks
that later tensors of the process are served from (``engine.state_placement``
and an INFO log line at ``initialize`` give the figures).  The placement
changes no result.

``stage3_gather_reuse`` (opt-in): at world size 1 a ZeRO-3 gather casts the
masters into the parameters every time, as minispeed does (stage_3.py:67-86),
1.3 ms at 1.3B params.  With the option the gather skips that cast when the
parameters' buffer already holds the cast of the current masters (nothing
has written the masters or the parameters since), which torch's version
counters tell, except for a write through a freed placeholder's ``.data``:
that one survives the next gather, where minispeed would overwrite it.
"""

from __future__ import annotations

import json
from typing import Any, Dict, Optional, Union

SUPPORTED_DTYPES = ("fp32", "fp16", "bf16")
SUPPORTED_OPTIMIZERS = ("AdamW", "Adam")
SUPPORTED_SCHEDULERS = ("WarmupDecayLR", "WarmupLR", "WarmupLRConst", "ConstantLR")

_TORCH_DTYPE_NAMES = {"fp32": "float32", "fp16": "float16", "bf16": "bfloat16"}


class ConfigError(ValueError):
    """An invalid or unsupported configuration (config.py:38-39)."""


def _section(raw: dict, key: str) -> dict:
    """A sub-dict of the config; ``None``/``False``/missing read as empty."""
    value = raw.get(key)
    return value if isinstance(value, dict) else {}


def _read(config: Union[dict, str, None]) -> dict:
    if config is None:
        return {}
    if isinstance(config, dict):
        return config
    if isinstance(config, str):
        with open(config, "r", encoding="utf-8") as fh:
            return json.load(fh)
    raise ConfigError(f"Unsupported config type: {type(config)}")


class DeepSpeedConfig:
    """Parsed and validated config (attribute names as in config.py:56-160)."""

    def __init__(self, config: Union[dict, str, None], world_size: int = 1):
        raw = _read(config)
        self.raw = raw
        self.world_size = world_size
        self._parse_batch(raw, world_size)
        self._parse_precision(raw)
        clip = raw.get("gradient_clipping")
        # 0 / missing / None disable clipping (config.py:101-102)
        self.gradient_clipping: Optional[float] = float(clip) if clip else None
        self._parse_zero(raw)
        self._parse_optimizer(raw)
        self._parse_scheduler(raw)
        self.steps_per_print = int(raw.get("steps_per_print", 10))
        self.seed = int(raw.get("seed", 1234))
        self.drop_overflow = bool(raw.get("drop_overflow_on_loss", True))
        hip = _section(raw, "hip_boundary")
        self.materialize_flat_grad = bool(hip.get("materialize_flat_grad", False))
        self.contiguous_gradients = bool(hip.get("contiguous_gradients", False))
        self.stage3_gather_reuse = bool(hip.get("stage3_gather_reuse", False))
        spacing = hip.get("state_spacing_gib", "auto")
        if spacing == "auto":
            self.state_spacing_bytes = -1          # flat.AUTO_SPACING
        elif spacing is None or isinstance(spacing, bool) or not isinstance(spacing, (int, float)) \
                or spacing < 0:
            raise ConfigError("hip_boundary.state_spacing_gib must be \"auto\" or a number >= 0, "
                              f"got {spacing!r}")
        else:
            self.state_spacing_bytes = int(float(spacing) * (1 << 30))

    # ------------------------------------------------------------ sections
    def _parse_batch(self, raw: dict, world: int) -> None:
        self.micro_batch = int(raw.get("train_micro_batch_size_per_gpu", 1))
        total = raw.get("train_batch_size")
        gas = raw.get("gradient_accumulation_steps")
        per_step = self.micro_batch * world
        if gas is None and total is not None:
            if total % per_step:
                raise ConfigError(
                    f"train_batch_size={total} is not divisible by "
                    f"micro_batch*world_size={per_step}"
                )
            gas = total // per_step
        self.gas = 1 if gas is None else int(gas)
        implied = per_step * self.gas
        if total is not None and int(total) != implied:
            raise ConfigError(
                f"train_batch_size={total} != micro_batch({self.micro_batch}) * "
                f"gas({self.gas}) * world_size({world}) = {implied}"
            )
        self.train_batch_size = implied

    def _parse_precision(self, raw: dict) -> None:
        fp16 = _section(raw, "fp16")
        bf16 = _section(raw, "bf16")
        explicit = raw.get("dtype")
        if explicit is not None:
            name = str(explicit).lower()
            if name not in SUPPORTED_DTYPES:
                raise ConfigError(f"dtype must be one of {SUPPORTED_DTYPES}")
            self.dtype = name
        elif fp16.get("enabled"):
            self.dtype = "fp16"
        elif bf16.get("enabled"):
            self.dtype = "bf16"
        else:
            self.dtype = "fp32"
        if fp16.get("enabled") and bf16.get("enabled"):
            raise ConfigError("fp16 and bf16 cannot both be enabled")
        self.fp16_enabled = self.dtype == "fp16"
        self.bf16_enabled = self.dtype == "bf16"
        self.loss_scale = float(fp16.get("loss_scale", 0.0))  # 0 => dynamic
        self.initial_scale_power = int(fp16.get("initial_scale_power", 16))
        self.loss_scale_window = int(fp16.get("loss_scale_window", 1000))
        self.scale_wrt_gas = bool(raw.get("scale_wrt_gas", True))

    def _parse_zero(self, raw: dict) -> None:
        zero = _section(raw, "zero_optimization")
        self.zero_stage = int(zero.get("stage", 0))
        if self.zero_stage not in (0, 1, 2, 3):
            raise ConfigError(
                f"Unsupported zero stage {self.zero_stage} (stages 0, 1, 2 and 3 exist)"
            )
        if zero.get("offload_optimizer") or zero.get("offload_param"):
            raise ConfigError("CPU/NVMe offload is not implemented")
        if zero.get("stage3_gather_16bit_weights_on_model_save") is False:
            raise ConfigError(
                "stage-3 parameters are always gathered on checkpoint save; set "
                "stage3_gather_16bit_weights_on_model_save to true or omit it"
            )

    def _parse_optimizer(self, raw: dict) -> None:
        opt = _section(raw, "optimizer")
        self.optimizer_type = str(opt.get("type", "AdamW"))
        if self.optimizer_type not in SUPPORTED_OPTIMIZERS:
            raise ConfigError(
                f"Unsupported optimizer '{self.optimizer_type}', "
                f"expected one of {SUPPORTED_OPTIMIZERS}"
            )
        params: Dict[str, Any] = dict(opt.get("params") or {})
        defaults = {"lr": 1e-3, "betas": (0.9, 0.999), "eps": 1e-8, "weight_decay": 0.0}
        for key, value in defaults.items():
            params.setdefault(key, value)
        params["betas"] = tuple(float(b) for b in params["betas"])
        self.optimizer_params = params

    def _parse_scheduler(self, raw: dict) -> None:
        sched = _section(raw, "scheduler")
        self.scheduler_type = str(sched.get("type", "WarmupLR"))
        if self.scheduler_type not in SUPPORTED_SCHEDULERS:
            raise ConfigError(
                f"Unsupported scheduler '{self.scheduler_type}', "
                f"expected one of {SUPPORTED_SCHEDULERS}"
            )
        params = dict(sched.get("params") or {})
        params.setdefault("warmup_num_steps", 0)
        # warmup_max_lr follows the optimizer lr unless given (config.py:151-153)
        params.setdefault("warmup_max_lr", float(self.optimizer_params["lr"]))
        params.setdefault("warmup_min_lr", 0.0)
        self.scheduler_params = params

    # ------------------------------------------------------------- helpers
    @property
    def torch_dtype(self):
        import torch

        return getattr(torch, _TORCH_DTYPE_NAMES[self.dtype])

    _SHOWN = ("dtype", "zero_stage", "gas", "micro_batch", "gradient_clipping",
              "state_spacing_bytes", "materialize_flat_grad", "contiguous_gradients",
              "stage3_gather_reuse")

    def __repr__(self) -> str:
        shown = ", ".join(f"{k}={getattr(self, k, None)!r}" for k in self._SHOWN)
        return f"{type(self).__name__}({shown})"


def load_config(
    config: Union[DeepSpeedConfig, dict, str, None], world_size: int = 1
) -> DeepSpeedConfig:
    if isinstance(config, DeepSpeedConfig):
        return config
    return DeepSpeedConfig(config, world_size=world_size)
