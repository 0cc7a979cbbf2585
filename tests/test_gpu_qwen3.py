"""The device-resident decode step (models/llm/qwen3.cpp:497-564) and its
ANE-contraction pieces on the GPU against the oracle: the RNE fp16 cast is
bit-exact; a projection (fp16 in, fp32 accumulation, fp16 out) is within
1 fp16 ulp of the exactly accumulated one plus the fp32-accumulation bound
(which matters only for outputs that cancel towards zero); the whole step's logits stay
within 4e-3 of the logit scale of the oracle's over 20 steps that wrap the
KV rings (the fp16 rounding points are where the two can part by an ulp)."""
import numpy as np
import pytest

from helpers import assert_bitexact, dev, host, save_qwen3, tiny_qwen3

pytestmark = pytest.mark.gpu


def test_f32_to_f16_rne_bitexact(hip, orc, rng):
    import torch

    bounds = np.arange(0, 0x7C01, dtype=np.uint32).astype(np.uint16).view(np.float16).astype(np.float32)
    mids = ((bounds[:-1].astype(np.float64) + bounds[1:]) / 2).astype(np.float32)
    x = np.concatenate([bounds, mids, np.nextafter(mids, np.float32(np.inf)), rng.standard_normal(100001).astype(np.float32),
                        np.array([65520.0, 1e30, np.inf, np.nan, 2 ** -25], np.float32)])
    x = np.concatenate([x, -x])
    out = torch.empty(x.size, dtype=torch.int16, device="cuda")
    hip.f32_to_f16(out, dev(x))
    got = host(out)
    want = orc.f32_to_f16_rne(x)
    nan = np.isnan(x)
    assert_bitexact(got[~nan], want[~nan], "f32_to_f16")
    assert np.all((got[nan] & 0x7C00) == 0x7C00) and np.all(got[nan] & 0x3FF)


@pytest.mark.parametrize("B,out_dim,in_dim", [(1, 4096, 1024), (64, 1024, 2048), (3, 77, 100), (17, 3072, 1024)])
def test_linear_f16_within_one_ulp(hip, orc, rng, B, out_dim, in_dim):
    import torch

    x = rng.standard_normal((B, in_dim)).astype(np.float16).view(np.uint16)
    w = (0.03 * rng.standard_normal((out_dim, in_dim))).astype(np.float16).view(np.uint16)
    y = torch.empty(B, out_dim, dtype=torch.int16, device="cuda")
    blas = hip.Blas()
    blas.linear_f16(y, dev(x), dev(w))
    got = host(y).view(np.float16).astype(np.float64)
    ref = orc.linear_f16(x, w).view(np.float16).astype(np.float64)
    # one fp16 ulp of the result, plus what an fp32 accumulation may differ
    # from the exact sum by (relative 2^-21 per term magnitude); outputs that
    # cancel towards zero have tiny ulps, so the second term matters there
    ulp = np.spacing(np.abs(ref).astype(np.float16)).astype(np.float64)
    mag = np.abs(x.view(np.float16).astype(np.float64)) @ np.abs(w.view(np.float16).astype(np.float64)).T
    assert np.all(np.abs(got - ref) <= ulp + mag * 2.0 ** -21 * 4)
    assert np.mean(got != ref) < 0.01


@pytest.mark.parametrize("B,out_dim,in_dim", [(1, 4096, 1024), (3, 1024, 3072), (8, 6144, 1024), (2, 77, 1000),
                                               (1, 151936, 1024), (5, 1024, 2048)])
def test_proj_f16_fused_conversions(hip, orc, rng, B, out_dim, in_dim):
    import torch

    x = rng.standard_normal((B, in_dim)).astype(np.float32)
    w = (0.03 * rng.standard_normal((out_dim, in_dim))).astype(np.float16).view(np.uint16)
    y = torch.empty(B, out_dim, device="cuda")
    hip.proj_f16(y, dev(x), dev(w))
    got = host(y).astype(np.float64)
    x16 = orc.f32_to_f16_rne(x).reshape(B, in_dim)
    ref = orc.linear_f16(x16, w).view(np.float16).astype(np.float64)
    assert np.array_equal(got.astype(np.float16).astype(np.float64), got)      # outputs are fp16 values
    ulp = np.spacing(np.abs(ref).astype(np.float16)).astype(np.float64)
    mag = np.abs(x16.view(np.float16).astype(np.float64)) @ np.abs(w.view(np.float16).astype(np.float64)).T
    assert np.all(np.abs(got - ref) <= ulp + mag * 2.0 ** -21 * 4)


@pytest.mark.parametrize("tied,B", [(True, 3), (False, 3), (True, 11)])
def test_decode_steps_match_oracle(hip, orc, rng, tmp_path, tied, B):
    import torch

    t, d = tiny_qwen3(rng, tied=tied)
    path = tmp_path / "tiny.safetensors"
    save_qwen3(path, t)
    cap, steps = 16, 20
    cfg = hip.Qwen3Config(d["H"], d["L"], d["nq"], d["nk"], d["D"], d["I"], d["V"], 1e6, 1e-6)
    ocfg = orc.Qwen3Config(d["H"], d["L"], d["nq"], d["nk"], d["D"], d["I"], d["V"], 1e6, 1e-6)
    model = hip.Qwen3Model(path, cfg, max_batch=B, kv_capacity=cap)
    ref = orc.Qwen3(ocfg, t, B, cap)
    logits = torch.empty(B, d["V"], device="cuda")
    pos0 = np.array([0, 100, 20000] * 4)[:B]    # every third sequence uses the RoPE fallback
    worst = 0.0
    for s in range(steps):
        ids = rng.integers(0, d["V"], B).astype(np.int32)
        pos = (pos0 + s).astype(np.int32)
        model.forward(dev(ids), dev(pos), logits)
        want = ref.forward(ids, pos)
        got = host(logits)
        err = np.max(np.abs(got - want), axis=1) / np.max(np.abs(want), axis=1)
        worst = max(worst, float(err.max()))
    assert worst < 4e-3, worst
    model.close()


def test_bad_config_and_missing_file(hip, tmp_path):
    cfg = hip.Qwen3Config(256, 2, 4, 2, 96, 384, 300, 1e6, 1e-6)          # head_dim 96 unsupported
    with pytest.raises(hip.AnelmError):
        hip.Qwen3Model(tmp_path / "x.safetensors", cfg, 1)
    cfg = hip.Qwen3Config(256, 2, 4, 2, 128, 384, 300, 1e6, 1e-6)
    with pytest.raises(hip.AnelmError):
        hip.Qwen3Model(tmp_path / "absent.safetensors", cfg, 1)
