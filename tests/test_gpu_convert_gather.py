"""bf16->fp16 convert (include/ane_lm/common.h:58-83) and embedding gather
(models/llm/qwen3.cpp:498) on the GPU: bit-exact against the oracle."""
import os

import numpy as np
import pytest

from helpers import assert_bitexact, dev, f16_normal, host

pytestmark = pytest.mark.gpu
GOLDEN = os.path.join(os.path.dirname(__file__), "golden")


def test_convert_exhaustive_patterns(hip, orc):
    import torch

    pats = np.arange(65536, dtype=np.uint16)
    src = dev(pats)
    dst = torch.empty_like(src)
    hip.bf16_to_f16(dst, src)
    got = host(dst)
    assert_bitexact(got, orc.bf16_to_f16(pats), "GPU vs oracle")
    assert_bitexact(got, np.load(os.path.join(GOLDEN, "bf16_to_f16_table.npy")), "GPU vs committed table")


@pytest.mark.parametrize("n,offset", [(10_000_003, 0), (8 * 4096 * 37, 0), (1, 0), (7, 0), (4096, 1), (999, 3)])
def test_convert_sizes_and_alignment(hip, orc, rng, n, offset):
    import torch

    bits = rng.integers(0, 65536, n + offset, dtype=np.uint32).astype(np.uint16)
    src = dev(bits)[offset:]
    dst = torch.empty(n + offset, dtype=torch.int16, device="cuda")[offset:]
    hip.bf16_to_f16(dst, src)
    assert_bitexact(host(dst), orc.bf16_to_f16(bits[offset:]), f"n={n} offset={offset}")


def test_convert_in_place(hip, orc, rng):
    bits = rng.integers(0, 65536, 1 << 20, dtype=np.uint32).astype(np.uint16)
    t = dev(bits)
    hip.bf16_to_f16(t, t)
    assert_bitexact(host(t), orc.bf16_to_f16(bits), "in place")


def _qwen3_8b_shapes():
    H, I, V, L, Dq, Dkv = 4096, 12288, 151936, 36, 4096, 1024
    shapes = [(V, H), (V, H), (H,)]
    for _ in range(L):
        shapes += [(Dq, H), (Dkv, H), (Dkv, H), (H, Dq), (I, H), (I, H), (H, I), (H,), (H,), (128,), (128,)]
    return shapes


@pytest.mark.slow
def test_convert_full_qwen3_8b_set(hip, orc):
    """The 8,190,735,360-parameter Qwen3-8B bf16 set, one call per tensor,
    then again in one call over the whole contiguous set (above 2^31
    elements, which one call of the reference's int-counted
    bf16_to_f16_vec, include/ane_lm/common.h:81-83, cannot take), each
    verified on the device against the oracle's 65,536-entry table."""
    import torch

    shapes = _qwen3_8b_shapes()
    n = sum(int(np.prod(s)) for s in shapes)
    assert n == 8_190_735_360
    g = torch.Generator(device="cuda").manual_seed(7)
    src = torch.empty(n, dtype=torch.int16, device="cuda")
    step = 1 << 28
    for i in range(0, n, step):  # ~N(0, 0.02) as truncated bf16, plus every pattern below
        m = min(step, n - i)
        f = torch.randn(m, generator=g, device="cuda", dtype=torch.float32) * 0.02
        src[i:i + m] = (f.view(torch.int32) >> 16).to(torch.int16)
    src[:65536] = torch.arange(65536, device="cuda", dtype=torch.int32).to(torch.int16)
    dst = torch.empty_like(src)
    off = 0
    for s in shapes:
        m = int(np.prod(s))
        hip.bf16_to_f16(dst[off:off + m], src[off:off + m])
        off += m
    lut = dev(orc.bf16_to_f16(np.arange(65536, dtype=np.uint16)))

    def mismatches():
        bad = 0
        for i in range(0, n, step):
            m = min(step, n - i)
            idx = src[i:i + m].to(torch.int32) & 0xFFFF
            bad += int((lut[idx] != dst[i:i + m]).sum().item())
        return bad

    assert mismatches() == 0, "one call per tensor"
    # one call over the whole set; 0x7FFF (an fp16 NaN, which the convert
    # never produces: NaN maps to infinity) marks anything left unwritten
    dst.fill_(0x7FFF)
    hip.bf16_to_f16(dst, src)
    assert mismatches() == 0, "one call over the contiguous set"


@pytest.mark.parametrize("hidden", [1024, 2560, 4096])
def test_gather_f16_table(hip, orc, rng, hidden):
    import torch

    V = 151936
    table = f16_normal(rng, (V, hidden), 0.02)
    ids = rng.integers(0, V, 64).astype(np.int32)
    ids[:3] = [0, V - 1, ids[3]]
    tt = dev(table).view(torch.float16)
    out = torch.empty(64, hidden, device="cuda")
    hip.embed_gather(out, tt, dev(ids))
    assert_bitexact(host(out), orc.embed_gather(table, ids, 1), f"hidden {hidden}")


def test_gather_every_f16_pattern(hip, orc):
    """Rows holding all 65,536 fp16 patterns (subnormals, Inf, NaN payloads)."""
    import torch

    table = np.arange(65536, dtype=np.uint16).reshape(64, 1024)
    ids = np.arange(64, dtype=np.int32)[::-1].copy()
    out = torch.empty(64, 1024, device="cuda")
    hip.embed_gather(out, dev(table).view(torch.float16), dev(ids))
    assert_bitexact(host(out), orc.embed_gather(table, ids, 1), "all fp16 patterns")


@pytest.mark.parametrize("dt", ["f32", "bf16"])
def test_gather_other_dtypes(hip, orc, rng, dt):
    import torch

    V, H = 5000, 1024
    if dt == "f32":
        table = rng.normal(0, 0.02, (V, H)).astype(np.float32)
        tt = dev(table)
        code = 0
    else:
        table = rng.integers(0, 65536, (V, H), dtype=np.uint32).astype(np.uint16)
        tt = dev(table).view(torch.bfloat16)
        code = 2
    ids = rng.integers(0, V, 17).astype(np.int32)
    out = torch.empty(17, H, device="cuda")
    hip.embed_gather(out, tt, dev(ids))
    assert_bitexact(host(out), orc.embed_gather(table, ids, code), dt)


def test_gather_ragged_hidden_and_bad_ids(hip, orc, rng):
    import torch

    V, H = 300, 1001
    table = f16_normal(rng, (V, H), 0.02)
    ids = np.array([5, -1, 299, 300, 7], np.int32)
    out = torch.full((5, H), 123.0, device="cuda")
    bad = torch.zeros(1, dtype=torch.int32, device="cuda")
    hip.embed_gather(out, dev(table).view(torch.float16), dev(ids), bad_count=bad)
    o = host(out)
    assert int(host(bad)[0]) == 2
    good = [0, 2, 4]
    assert_bitexact(o[good], orc.embed_gather(table, ids[good], 1), "good rows")
    assert np.all(o[[1, 3]] == 123.0), "rows with bad ids must not be written"


@pytest.mark.parametrize("n", [65536, 4096, 1, 3_000_017])
def test_norm_weight_plus1(hip, orc, rng, n):
    """Qwen3.5 (1+w) norm weight (core/safetensors.cpp:299-306): bit-exact with
    the oracle over all 65,536 bf16 patterns (NaN payloads included) and at
    ragged sizes."""
    import torch

    pats = np.arange(65536, dtype=np.uint16) if n == 65536 else rng.integers(0, 65536, n, dtype=np.uint32).astype(np.uint16)
    dst = torch.empty(n, device="cuda")
    hip.bf16_to_f32_plus1(dst, dev(pats))
    assert_bitexact(host(dst), orc.norm_weight(pats), f"n={n}")


def test_convert_many_tensors_one_call(hip, orc, rng):
    """anelm_bf16_to_f16_multi: 300 tensors (three launches of up to 128),
    sizes 1 .. 70,000 including tails that are not a multiple of 8, empty
    tensors, one in place and two not 16-byte aligned (own launches); every
    output bit-exact, and the bytes between tensors untouched."""
    import torch

    sizes = [int(x) for x in rng.integers(1, 70_000, 300)]
    sizes[:6] = [1, 7, 8, 4096, 4097, 0]
    pad = 64                                      # untouched gap (elements) after each tensor
    offs = np.cumsum([0] + [((m + 7) // 8) * 8 + pad for m in sizes])
    bits = rng.integers(0, 65536, int(offs[-1]), dtype=np.uint32).astype(np.uint16)
    src = dev(bits)
    out = torch.full((int(offs[-1]),), 0x5A5A, dtype=torch.int16, device="cuda")
    srcs = [src[o:o + m] for o, m in zip(offs[:-1], sizes)]
    dsts = [out[o:o + m] for o, m in zip(offs[:-1], sizes)]
    dsts[10] = srcs[10]                           # in place
    srcs[20], dsts[20] = src[offs[20] + 1:offs[20] + 1 + sizes[20]], out[offs[20] + 3:offs[20] + 3 + sizes[20]]
    hip.bf16_to_f16_multi(dsts, srcs)
    got_out, got_src = host(out), host(src)
    for i, (o, m) in enumerate(zip(offs[:-1], sizes)):
        if i == 20:
            assert_bitexact(got_out[o + 3:o + 3 + m], orc.bf16_to_f16(bits[o + 1:o + 1 + m]), "unaligned tensor")
            continue
        ref = orc.bf16_to_f16(bits[o:o + m])
        assert_bitexact((got_src if i == 10 else got_out)[o:o + m], ref, f"tensor {i} ({m} elements)")
        if i not in (10, 20):
            assert np.all(got_out[o + m:int(offs[i + 1])].view(np.uint16) == 0x5A5A), f"gap after tensor {i}"


@pytest.mark.parametrize("n,offset", [(65536, 0), (8 * 1000, 0), (1, 0), (13, 0), (8 * 777, 2), (3_000_000, 0)])
@pytest.mark.parametrize("kind", ["f16", "bf16"])
def test_widen_to_f32(hip, orc, rng, n, offset, kind):
    """fp16 -> fp32 (common.h:35-56) and bf16 -> fp32 (common.h:21-26): exact,
    NaN payloads kept; the 8-wide path (aligned, n % 8 == 0) and the
    element-wise one (ragged or misaligned)."""
    import torch

    bits = np.arange(65536, dtype=np.uint16) if n == 65536 else rng.integers(0, 65536, n, dtype=np.uint32).astype(np.uint16)
    src = dev(np.concatenate([np.zeros(offset, np.uint16), bits]))[offset:]
    dst = torch.empty(n + offset, device="cuda")[offset:]
    (hip.f16_to_f32 if kind == "f16" else hip.bf16_to_f32)(dst, src)
    want = orc.f16_to_f32(bits) if kind == "f16" else orc.bf16_to_f32(bits)
    assert_bitexact(host(dst), want, f"{kind} n={n} offset={offset}")
