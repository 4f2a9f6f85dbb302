"""Host-side logic on the CPU: config schema, loss-scale state machine, LR
schedules, param-group normalisation, single-GPU guards.

The known-answer values are the ones minispeed's own tests assert
(tests/test_config.py:6-77, tests/test_precision.py:14-70); the scaler and
schedule KATs run against both this package and the oracle.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch
from torch import nn

import minispeed_amd as ms
from minispeed_amd import comm
from minispeed_amd.config import ConfigError, DeepSpeedConfig
from minispeed_amd.engine import _normalize_param_groups
from minispeed_amd.optim.scheduler import WarmupDecayLR, WarmupLR, build_scheduler
from minispeed_amd.precision import DynamicLossScaler
from oracle import boundary as ob


# ------------------------------------------------------------------ config
def test_gas_derived_from_train_batch_size():
    cfg = DeepSpeedConfig({"train_batch_size": 32, "train_micro_batch_size_per_gpu": 8}, world_size=2)
    assert cfg.gas == 2 and cfg.train_batch_size == 32


def test_inconsistent_batch_sizes_raise():
    with pytest.raises(ConfigError):
        DeepSpeedConfig({"train_batch_size": 33, "train_micro_batch_size_per_gpu": 8}, world_size=2)
    with pytest.raises(ConfigError):
        DeepSpeedConfig({"train_batch_size": 32, "train_micro_batch_size_per_gpu": 8,
                         "gradient_accumulation_steps": 3}, world_size=1)


def test_dtype_resolution():
    assert DeepSpeedConfig({}).dtype == "fp32"
    assert DeepSpeedConfig({"fp16": {"enabled": True}}).dtype == "fp16"
    assert DeepSpeedConfig({"bf16": {"enabled": True}}).dtype == "bf16"
    assert DeepSpeedConfig({"dtype": "bf16"}).dtype == "bf16"
    assert DeepSpeedConfig({"dtype": "BF16"}).dtype == "bf16"
    with pytest.raises(ConfigError):
        DeepSpeedConfig({"dtype": "fp8"})


def test_fp16_and_bf16_conflict():
    with pytest.raises(ConfigError):
        DeepSpeedConfig({"fp16": {"enabled": True}, "bf16": {"enabled": True}})


def test_zero_stage_validation():
    assert DeepSpeedConfig({"zero_optimization": {"stage": 1}}).zero_stage == 1
    assert DeepSpeedConfig({"zero_optimization": {"stage": 3}}).zero_stage == 3
    with pytest.raises(ConfigError):
        DeepSpeedConfig({"zero_optimization": {"stage": 4}})
    with pytest.raises(ConfigError):
        DeepSpeedConfig({"zero_optimization": {"stage": 1, "offload_optimizer": {"device": "cpu"}}})
    with pytest.raises(ConfigError):
        DeepSpeedConfig({"zero_optimization": {"stage": 3, "stage3_gather_16bit_weights_on_model_save": False}})


def test_defaults_and_clip_and_scaler_keys():
    cfg = DeepSpeedConfig({"optimizer": {"type": "AdamW", "params": {"lr": 3e-4}}})
    assert cfg.scheduler_params["warmup_max_lr"] == 3e-4
    assert cfg.optimizer_params["betas"] == (0.9, 0.999)
    assert cfg.optimizer_params["eps"] == 1e-8 and cfg.optimizer_params["weight_decay"] == 0.0
    assert cfg.gradient_clipping is None
    assert DeepSpeedConfig({"gradient_clipping": 0}).gradient_clipping is None
    assert DeepSpeedConfig({"gradient_clipping": 1}).gradient_clipping == 1.0
    f = DeepSpeedConfig({"fp16": {"enabled": True, "loss_scale": 128, "loss_scale_window": 50}})
    assert (f.loss_scale, f.initial_scale_power, f.loss_scale_window) == (128.0, 16, 50)
    assert DeepSpeedConfig({"optimizer": {"type": "Adam"}}).optimizer_type == "Adam"
    with pytest.raises(ConfigError):
        DeepSpeedConfig({"optimizer": {"type": "SGD"}})
    with pytest.raises(ConfigError):
        DeepSpeedConfig({"scheduler": {"type": "OneCycle"}})
    assert DeepSpeedConfig({"hip_boundary": {"materialize_flat_grad": True}}).materialize_flat_grad
    assert not DeepSpeedConfig({}).materialize_flat_grad
    assert DeepSpeedConfig({}).state_spacing_bytes == -1            # auto
    assert DeepSpeedConfig({"hip_boundary": {"state_spacing_gib": "auto"}}).state_spacing_bytes == -1
    assert DeepSpeedConfig({"hip_boundary": {"state_spacing_gib": 0}}).state_spacing_bytes == 0
    assert DeepSpeedConfig({"hip_boundary": {"state_spacing_gib": 32}}).state_spacing_bytes == 32 << 30
    assert DeepSpeedConfig({"hip_boundary": {"state_spacing_gib": 1.5}}).state_spacing_bytes == 3 << 29
    for bad in (-1, "32", "Auto", True, None):
        with pytest.raises(ConfigError):
            DeepSpeedConfig({"hip_boundary": {"state_spacing_gib": bad}})


def test_config_from_json_file(tmp_path):
    path = tmp_path / "ds.json"
    path.write_text('{"train_micro_batch_size_per_gpu": 4, "gradient_accumulation_steps": 2, "dtype": "bf16"}')
    cfg = DeepSpeedConfig(str(path))
    assert (cfg.micro_batch, cfg.gas, cfg.dtype) == (4, 2, "bf16")
    with pytest.raises(ConfigError):
        DeepSpeedConfig(42)


# ------------------------------------------------------------------ scaler
SCALERS = [DynamicLossScaler, ob.LossScaler]


@pytest.mark.parametrize("cls", SCALERS)
def test_scaler_grows_after_window(cls):
    s = cls(enabled=True, init_scale=8.0, scale_window=3)
    for _ in range(3):
        s.update(overflow=False)
    assert s.scale == 16.0


@pytest.mark.parametrize("cls", SCALERS)
def test_scaler_halves_on_overflow_and_resets_window(cls):
    s = cls(enabled=True, init_scale=16.0, scale_window=2)
    s.update(overflow=False)
    s.update(overflow=True)
    assert (s.scale, s.skipped_steps, s.good_steps) == (8.0, 1, 0)
    s.update(overflow=False)
    assert s.scale == 8.0
    s.update(overflow=False)
    assert s.scale == 16.0


@pytest.mark.parametrize("cls", SCALERS)
def test_scaler_disabled_is_noop(cls):
    s = cls(enabled=False)
    assert s.loss_scale_factor == 1.0
    s.update(overflow=True)
    assert s.scale == 1.0


@pytest.mark.parametrize("cls", SCALERS)
def test_scaler_floor_ceiling_and_static_start(cls):
    s = cls(enabled=True, init_scale=2.0, scale_window=1)
    s.update(True)
    s.update(True)
    assert s.scale == 1.0 and s.skipped_steps == 2          # floor at min_scale
    s = cls(enabled=True, init_scale=2.0 ** 24, scale_window=1)
    s.update(False)
    assert s.scale == 2.0 ** 24 and s.good_steps == 1       # ceiling: no growth, no reset
    s = cls(enabled=True, init_scale=1000.0, scale_window=1)
    s.update(False)
    assert s.scale == 2000.0                                 # a static value stays dynamic
    s = cls(enabled=True)
    s.set_scale_from_power(16)
    assert s.scale == 65536.0


def test_scaler_state_dict_roundtrip():
    s = DynamicLossScaler(enabled=True, init_scale=64.0, scale_window=5)
    s.update(False)
    s.update(True)
    t = DynamicLossScaler(enabled=True)
    t.load_state_dict(s.state_dict())
    assert t.state_dict() == s.state_dict()


# --------------------------------------------------------------- schedules
class _Opt:
    def __init__(self, lr=0.0, n=1):
        self.param_groups = [{"lr": lr} for _ in range(n)]


def _oracle_sched(kind, **kw):
    opt = _Opt()
    return opt, ob.Schedule(opt.param_groups, kind, kw.get("warmup_min_lr", 0.0),
                            kw["warmup_max_lr"], kw.get("warmup_num_steps", 0),
                            kw.get("total_num_steps"))


@pytest.mark.parametrize("impl", ["package", "oracle"])
def test_warmup_lr_schedule(impl):
    kw = dict(warmup_min_lr=0.0, warmup_max_lr=1.0, warmup_num_steps=4)
    if impl == "package":
        sched = WarmupLR(_Opt(), **kw)
    else:
        _, sched = _oracle_sched("WarmupLR", **kw)
    lrs = []
    for _ in range(6):
        sched.step()
        lrs.append(sched.get_last_lr())
    assert lrs == [0.0, 0.25, 0.5, 0.75, 1.0, 1.0]


@pytest.mark.parametrize("impl", ["package", "oracle"])
def test_warmup_decay_lr_schedule(impl):
    kw = dict(warmup_min_lr=0.0, warmup_max_lr=1.0, warmup_num_steps=2, total_num_steps=6)
    if impl == "package":
        sched = WarmupDecayLR(_Opt(), **kw)
    else:
        _, sched = _oracle_sched("WarmupDecayLR", **kw)
    lrs = []
    for _ in range(7):
        sched.step()
        lrs.append(round(sched.get_last_lr(), 6))
    assert lrs == [0.0, 0.5, 1.0, 0.75, 0.5, 0.25, 0.0]


def test_schedule_writes_every_group_and_builds_by_name():
    opt = _Opt(lr=0.3, n=3)
    sched = build_scheduler(opt, "WarmupDecayLR", {"warmup_max_lr": 1.0, "warmup_num_steps": 0,
                                                   "total_num_steps": 4})
    assert [g["lr"] for g in opt.param_groups] == [0.3] * 3   # not stepped at construction
    sched.step()
    assert [g["lr"] for g in opt.param_groups] == [1.0] * 3
    assert isinstance(build_scheduler(_Opt(), "ConstantLR", {"warmup_max_lr": 1.0}), WarmupLR)
    with pytest.raises(ValueError):
        build_scheduler(_Opt(), "Cosine", {})
    st = sched.state_dict()
    other = build_scheduler(_Opt(), "WarmupDecayLR", {"warmup_max_lr": 1.0, "total_num_steps": 4})
    other.load_state_dict(st)
    assert other.last_epoch == sched.last_epoch == 0


# ------------------------------------------------------- engine host glue
def test_normalize_param_groups_forms():
    m = nn.Sequential(nn.Linear(2, 3), nn.Linear(3, 1))
    frozen = nn.Parameter(torch.zeros(2), requires_grad=False)
    defaults = {"lr": 1e-3, "weight_decay": 0.1}
    g = _normalize_param_groups(m, None, defaults)
    assert len(g) == 1 and len(g[0]["params"]) == 4 and g[0]["lr"] == 1e-3
    g = _normalize_param_groups(m, list(m.parameters()) + [frozen], defaults)
    assert len(g[0]["params"]) == 4
    g = _normalize_param_groups(m, [{"params": list(m[0].parameters()), "lr": 5.0},
                                    {"params": list(m[1].parameters())},
                                    {"params": [frozen]}], defaults)
    assert [x["lr"] for x in g] == [5.0, 1e-3] and g[0]["weight_decay"] == 0.1
    g = _normalize_param_groups(m, {"params": list(m[1].parameters()), "eps": 1.0}, defaults)
    assert g[0]["eps"] == 1.0 and len(g[0]["params"]) == 2
    with pytest.raises(ValueError):
        _normalize_param_groups(m, [frozen], defaults)


def test_initialize_requires_model_and_single_rank(monkeypatch):
    with pytest.raises(ValueError):
        ms.initialize(model=None)
    monkeypatch.setenv("WORLD_SIZE", "2")
    monkeypatch.setenv("RANK", "0")
    with pytest.raises(comm.MultiGPUNotSupported):
        ms.initialize(model=nn.Linear(2, 2), config={})


def test_engine_refuses_a_cpu_device(monkeypatch):
    monkeypatch.setenv("MINISPEED_DEVICE", "cpu")
    with pytest.raises(RuntimeError, match="HIP"):
        ms.initialize(model=nn.Linear(2, 2), config={})


def test_world_one_collectives_are_identities():
    t = torch.arange(4.0)
    assert comm.all_reduce(t) is t and comm.broadcast(t) is t
    assert comm.all_reduce_flag(True) is True and comm.all_reduce_flag(False) is False
    out = torch.zeros(4)
    comm.reduce_scatter(out, t)
    assert torch.equal(out, t)
    out2 = torch.zeros(4)
    comm.all_gather_flat(out2, t)
    assert torch.equal(out2, t)
    assert comm.get_world_size() == 1 and comm.get_rank() == 0 and not comm.is_distributed()


def test_timers_accumulate():
    t = ms.Timers()
    with t.timer("step"):
        pass
    assert t.names() == ["step"] and t("step").elapsed >= 0.0
    assert "step:" in t.log()
    t.reset()
    assert t("step").elapsed == 0.0
    # minispeed's Timer carries started_at (utils.py:18): None while idle,
    # the start of the outermost open section otherwise; settable as there
    timer = t("io")
    assert timer.started_at is None
    with timer.section():
        outer = timer.started_at
        assert outer is not None
        with timer:
            assert timer.started_at == outer
        assert timer.started_at == outer
    assert timer.started_at is None and timer.elapsed > 0.0
    timer.started_at = 1.0
    assert timer.started_at == 1.0


def test_scale_transition_equals_the_oracle_scaler_on_random_runs():
    """The package's pure transition function and the oracle's scaler (the
    reference's state machine restated, pinned by minispeed's own recorded
    trajectories) walk the same (scale, good, skipped) path."""
    from minispeed_amd.precision import ScaleState, scale_transition

    rng = np.random.default_rng(3)
    for trial in range(200):
        window = int(rng.integers(1, 6))
        start = float(2.0 ** int(rng.integers(0, 26)))
        ref = ob.LossScaler(enabled=True, init_scale=start, scale_window=window)
        state = ScaleState(start, 0, 0)
        for overflow in rng.random(60) < rng.random():
            ref.update(bool(overflow))
            state = scale_transition(state, bool(overflow), window=window, min_scale=1.0,
                                     max_scale=2.0 ** 24)
            assert state == (ref.scale, ref.good_steps, ref.skipped_steps), trial


def test_schedule_functions_equal_the_oracle_schedule_bit_for_bit():
    from minispeed_amd.optim.scheduler import WarmupSpec, warmup_decay_lr, warmup_lr

    rng = np.random.default_rng(4)
    for trial in range(100):
        lo, hi = sorted(float(x) for x in rng.random(2) * 1e-2)
        warm = int(rng.integers(-2, 50))
        total = None if trial % 7 == 0 else warm + int(rng.integers(-5, 200))
        for kind, fn in (("WarmupLR", warmup_lr), ("WarmupDecayLR", warmup_decay_lr)):
            groups = [{"lr": 0.0}]
            ref = ob.Schedule(groups, kind, lo, hi, warm, total)
            spec = WarmupSpec(lo, hi, max(0, warm), total)
            for e in range(-1, 260):
                ref.last_epoch = e
                assert fn(spec, e) == ref.get_lr(), (trial, kind, e)


# ------------------------------------------------------ K2's host read-back
def _readback(patience):
    """A HostReadback over ordinary host memory (pinned memory needs a GPU;
    the polling logic does not)."""
    from minispeed_amd import _native
    from minispeed_amd.boundary import HostReadback

    rb = object.__new__(HostReadback)
    rb.host = torch.zeros(_native.SCALARS_BYTES, dtype=torch.uint8)
    rb._bytes = rb.host.numpy()
    rb._ready = rb._bytes[HostReadback._READY:HostReadback._READY + 4].view(np.uint32)
    rb.patience = patience
    return rb


def test_host_readback_returns_once_the_ready_word_turns():
    """wait() spins until the kernel's ready word is 1 and then returns the
    struct the kernel wrote before it; arm() clears the word."""
    import threading
    import time

    from minispeed_amd import _native

    rb = _readback(patience=30.0)
    rb._ready[0] = 1
    rb.arm()
    assert rb._ready[0] == 0
    want = _native.StepScalars(overflow=0, clip_applied=1, sumsq=4.0, norm=2.0, coef=0.5, ready=0,
                               coef64=0.5, next_scale=1024.0, next_good_steps=3, next_skipped_steps=1)

    def kernel():
        time.sleep(0.05)
        raw = np.frombuffer(bytes(want), dtype=np.uint8)
        rb._bytes[:] = raw
        rb._ready[0] = 1                          # the word last, as K2 sets it

    t = threading.Thread(target=kernel)
    t.start()
    got = rb.wait(stream=0)
    t.join()
    assert (got.ready, got.clip_applied, got.norm, got.coef64, got.next_scale, got.next_good_steps) == \
        (1, 1, 2.0, 0.5, 1024.0, 3)


def test_host_readback_falls_back_to_a_stream_sync_and_raises_if_nothing_arrived(monkeypatch):
    """Past its patience wait() synchronises the stream (which also reports a
    device error) and raises when the word is still not set; if the word
    arrives with the synchronisation, the struct is returned."""
    from minispeed_amd import _native

    calls = []

    class FakeHip:
        def __init__(self, on_sync=None):
            self.on_sync = on_sync

        def hipStreamSynchronize(self, stream):
            calls.append(stream)
            if self.on_sync:
                self.on_sync()
            return 0

    rb = _readback(patience=0.02)
    rb.arm()
    monkeypatch.setattr(_native, "hip_runtime", lambda: FakeHip())
    with pytest.raises(RuntimeError, match="did not arrive"):
        rb.wait(stream=77)
    assert calls == [77]

    rb.arm()

    def land():
        rb._ready[0] = 1

    monkeypatch.setattr(_native, "hip_runtime", lambda: FakeHip(on_sync=land))
    assert rb.wait(stream=78).ready == 1
    assert calls == [77, 78]
