"""bench.py's host side on the CPU: the refusals that come before any device
work, the engine config it drives, its byte accounting and the measured
traffic it reports."""

from __future__ import annotations

import json

import pytest

import bench
from minispeed_amd.config import DeepSpeedConfig


def _error(capsys, argv):
    rc = bench.main(argv)
    out = capsys.readouterr().out.strip().splitlines()
    assert rc == 2 and len(out) == 1
    return json.loads(out[0])["error"]


@pytest.mark.parametrize("n", [2, 8])
def test_more_than_one_gpu_is_refused_with_a_message(capsys, n):
    msg = _error(capsys, ["--gpus", str(n)])
    assert f"--gpus {n}" in msg and "one GPU" in msg


@pytest.mark.parametrize("mode", ["fused", "materialize"])
def test_micro_batches_apply_to_contiguous_mode_only(capsys, mode):
    msg = _error(capsys, ["--mode", mode, "--micro-batches", "4"])
    assert "--mode contiguous" in msg
    assert "--mode contiguous" in _error(capsys, ["--mode", "contiguous", "--micro-batches", "0"])


def test_defaults_are_the_headline_workload():
    args = bench.parse([])
    assert (args.gpus, args.workload, args.grad_dtype, args.mode, args.zero_stage,
            args.state_spacing_gib, args.micro_batches) == (1, "gpt-1.3b", "fp16", "fused", 1,
                                                           "auto", 1)
    assert args.steps >= 20 and args.warmup >= 5


@pytest.mark.parametrize("dtype", ["fp16", "bf16", "fp32"])
@pytest.mark.parametrize("mode", ["fused", "materialize", "contiguous"])
def test_engine_config_parses_to_the_workload(dtype, mode):
    cfg = DeepSpeedConfig(bench.engine_config(dtype, mode, 3, 0, gas=4))
    assert cfg.dtype == dtype and cfg.zero_stage == 3 and cfg.gas == 4
    assert cfg.gradient_clipping == 1.0
    assert cfg.materialize_flat_grad == (mode == "materialize")
    assert cfg.contiguous_gradients == (mode == "contiguous")
    assert cfg.state_spacing_bytes == 0
    assert DeepSpeedConfig(bench.engine_config(dtype, mode, 3, 0, gather_reuse=True)).stage3_gather_reuse
    if dtype == "fp16":              # dynamic loss scale from 2^16
        assert cfg.loss_scale == 0.0 and cfg.initial_scale_power == 16
    assert DeepSpeedConfig(bench.engine_config(dtype, mode)).state_spacing_bytes == -1


def test_byte_accounting_per_mode():
    # K1 + K3 bytes per parameter: the fused step re-reads the half
    # gradients (30), the materialized one writes and reads fp32 (36), the
    # contiguous one reads the fp32 sums the hooks left (30)
    totals = {key: sum(v) for key, v in bench.BYTES.items()}
    assert totals == {("fused", 2): 30, ("materialize", 2): 36, ("fused", 4): 36,
                      ("materialize", 4): 40, ("contiguous", 2): 30, ("contiguous", 4): 30}


def test_measured_traffic_only_for_the_measured_configuration():
    k3 = bench.traffic_for("k3", "gpt-1.3b", "fp16", "fused", 36)
    assert k3 == bench.MEASURED_TRAFFIC["k3/gpt-1.3b/fp16/fused/36.0"]
    # 28 B/param: the counted traffic is the algorithmic traffic to 0.1%
    assert abs(k3 / (28 * 1_315_723_264) - 1) < 1e-3
    for other in (("k3", "gpt-1.3b", "fp16", "fused", 0), ("k3", "gpt-1.3b", "fp16", "fused", 32),
                  ("k3", "gpt-1.3b", "bf16", "fused", 36),
                  ("k3", "gpt-1.3b", "fp16", "materialize", 36),
                  ("k3", "gpt2-124m", "fp16", "fused", 36)):
        assert bench.traffic_for(*other) is None


def test_shifted_workload_is_the_headline_list_behind_three_elements():
    from minispeed_amd.workloads import numel, shapes_of

    base, shifted = shapes_of("gpt-1.3b"), shapes_of("gpt-1.3b-shift3")
    assert shifted[0] == (3,) and shifted[1:] == base
    assert numel(shifted) == numel(base) + 3 == 1_315_723_267
    # every later tensor starts 3 elements past a multiple of 8 of the flat space
    off = 3
    for s in shifted[1:]:
        assert off % 8 == 3
        n = 1
        for x in s:
            n *= x
        off += n
