"""The device-resident decode step (models/llm/qwen3.cpp:497-564) and its
ANE-contraction pieces on the GPU against the oracle: the RNE fp16 cast is
bit-exact; a projection (fp16 in, fp32 accumulation, fp16 out) is within
1 fp16 ulp of the exactly accumulated one plus the fp32-accumulation bound
(which matters only for outputs that cancel towards zero); the whole step's logits stay
within 4e-3 of the logit scale of the oracle's over 20 steps that wrap the
KV rings (the fp16 rounding points are where the two can part by an ulp)."""
import numpy as np
import pytest

from helpers import assert_bitexact, bf16, dev, from_bf16, host, save_qwen3, tiny_qwen3

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


@pytest.mark.parametrize("B,out_dim,in_dim", [(1, 4096, 1024), (64, 1024, 2048), (3, 77, 100), (17, 3072, 1024),
                                               (64, 151936, 1024), (20, 70000, 256)])
def test_linear_f16_within_one_ulp(hip, orc, rng, B, out_dim, in_dim):
    import torch

    x = rng.standard_normal((B, in_dim)).astype(np.float16).view(np.uint16)
    w = (0.03 * rng.standard_normal((out_dim, in_dim))).astype(np.float16).view(np.uint16)
    y = torch.empty(B, out_dim, dtype=torch.int16, device="cuda")
    hip.linear_f16(y, dev(x), dev(w))
    got = host(y).view(np.float16).astype(np.float64)
    ref = orc.linear_f16(x, w).view(np.float16).astype(np.float64)
    # one fp16 ulp of the result, plus what an fp32 accumulation may differ
    # from the exact sum by (relative 2^-21 per term magnitude); outputs that
    # cancel towards zero have tiny ulps, so the second term matters there
    ulp = np.spacing(np.abs(ref).astype(np.float16)).astype(np.float64)
    mag = np.abs(x.view(np.float16).astype(np.float64)) @ np.abs(w.view(np.float16).astype(np.float64)).T
    assert np.all(np.abs(got - ref) <= ulp + mag * 2.0 ** -21 * 4)
    assert np.mean(got != ref) < 0.01


def check_projection(orc, x, w, got):
    """got (float64 of the fp32 outputs) against the oracle's fp16 projection:
    the outputs are fp16 values, within one fp16 ulp of the exactly rounded
    result plus what an fp32 accumulation may differ from the exact sum by."""
    B, in_dim = x.shape
    x16 = orc.f32_to_f16_rne(x).reshape(B, in_dim)
    ref = orc.linear_f16(x16, w).view(np.float16).astype(np.float64)
    assert np.array_equal(got.astype(np.float16).astype(np.float64), got)      # outputs are fp16 values
    ulp = np.spacing(np.abs(ref).astype(np.float16)).astype(np.float64)
    mag = np.abs(x16.view(np.float16).astype(np.float64)) @ np.abs(w.view(np.float16).astype(np.float64)).T
    assert np.all(np.abs(got - ref) <= ulp + mag * 2.0 ** -21 * 4)


# One or two rows of x (up to eight for out_dim <= 1024) take the dot kernel,
# the rest the MFMA kernel; in_dim not a multiple of 32 needs the dot kernel.
# The dot kernel's launch shapes: one output row per wave (1024-input rows in
# one round of loads, longer ones in rounds of 4 or 6 chunks, 4096 inputs in
# two rounds), two per wave from 4096 rows (odd counts leave a half-used
# wave), four from 32768 rows, and ragged in_dim (masked lanes).
@pytest.mark.parametrize("B,out_dim,in_dim", [(1, 4096, 1024), (3, 1024, 3072), (8, 6144, 1024), (2, 77, 1000),
                                               (1, 151936, 1024), (5, 1024, 2048), (16, 1000, 96), (17, 3072, 1024),
                                               (64, 4096, 1024), (33, 100, 32), (4, 64, 1000), (1, 4097, 1024),
                                               (2, 4101, 992), (1, 32771, 512), (1, 1023, 4096), (2, 1000, 2056),
                                               (8, 1024, 200), (1, 33, 8)])
def test_proj_f16_fused_conversions(hip, orc, rng, B, out_dim, in_dim):
    import torch

    x = rng.standard_normal((B, in_dim)).astype(np.float32)
    w = (0.03 * rng.standard_normal((out_dim, in_dim))).astype(np.float16).view(np.uint16)
    y = torch.empty(B, out_dim, device="cuda")
    hip.proj_f16(y, dev(x), dev(w))
    check_projection(orc, x, w, host(y).astype(np.float64))


@pytest.mark.parametrize("B,out_dim,in_dim", [(64, 1024, 3072), (40, 6144, 1024), (17, 2560, 9728),
                                               (64, 151936, 1024), (1, 48, 64), (33, 100, 32)])
def test_proj_f16_x16_inputs(hip, orc, rng, B, out_dim, in_dim):
    """Inputs rounded to fp16 beforehand (the oracle's RNE convert) give the
    same projection as fp32 inputs rounded inside; two calls in a row, the
    second with a smaller batch."""
    import torch

    w = (0.03 * rng.standard_normal((out_dim, in_dim))).astype(np.float16).view(np.uint16)
    dw = dev(w)
    for b in (B, max(1, B // 3)):
        x = rng.standard_normal((b, in_dim)).astype(np.float32)
        x16 = dev(orc.f32_to_f16_rne(x).reshape(b, in_dim).view(np.int16))
        y = torch.full((b, out_dim), float("nan"), device="cuda")
        hip.proj_f16_x16(y, x16, dw)
        check_projection(orc, x, w, host(y).astype(np.float64))


@pytest.mark.parametrize("B,out_dim,in_dim", [(17, 4096, 1024), (64, 1024, 2048), (40, 3072, 1024), (64, 1000, 96)])
@pytest.mark.parametrize("norm", [False, True])
def test_proj_f16_fused_past_16_rows(hip, orc, rng, B, out_dim, in_dim, norm):
    """The fp32-input fused projection past 16 rows (two batch blocks per
    workgroup with the norm prologue over 32 rows), store and residual add."""
    import torch

    x = (2 * rng.standard_normal((B, in_dim))).astype(np.float32)
    gamma = bf16(1 + 0.1 * rng.standard_normal(in_dim))
    w = (0.03 * rng.standard_normal((out_dim, in_dim))).astype(np.float16).view(np.uint16)
    y = torch.full((B, out_dim), float("nan"), device="cuda")
    g = dev(gamma.view(np.int16)) if norm else None
    hip.proj_f16_fused(y, dev(x), dev(w), norm=g, eps=1e-6)
    xn = np.stack([orc.rmsnorm(x[b], from_bf16(gamma), 1e-6) for b in range(B)]) if norm else x
    check_projection(orc, xn, w, host(y).astype(np.float64))
    r0 = rng.standard_normal((B, out_dim)).astype(np.float32)
    y = dev(r0)
    hip.proj_f16_fused(y, dev(x), dev(w), norm=g, eps=1e-6, epilogue=hip.PROJ_ADD)
    ref, mag = _proj_ref(orc, xn, w)
    want = r0.astype(np.float64) + ref
    tol = _ulp16(ref) + mag * 2.0 ** -21 * 4 + np.spacing(np.abs(want).astype(np.float32))
    assert np.all(np.abs(host(y).astype(np.float64) - want) <= tol)


@pytest.mark.parametrize("B,out_dim,in_dim", [(17, 4096, 1024), (64, 1024, 3072), (3, 1024, 2048), (64, 160, 64),
                                               (40, 512, 256), (100, 2048, 1024), (1, 6144, 1024), (2, 1024, 3072),
                                               (1, 40000, 1024), (1, 4096, 1024), (8, 1024, 4096), (1, 1000, 4128)])
def test_proj_f16_x16_fused_epilogues(hip, orc, rng, B, out_dim, in_dim):
    """fp16 rows in (the fp16 RMSNorm's output), each epilogue: store and
    residual add against the oracle, the SwiGLU in fp32 and rounded to fp16
    (the down projection's input), the latter bit-identical to the fp32
    SwiGLU narrowed."""
    import torch

    x = (2 * rng.standard_normal((B, in_dim))).astype(np.float32)
    x16 = dev(orc.f32_to_f16_rne(x).reshape(B, in_dim).view(np.int16))
    w = (0.03 * rng.standard_normal((out_dim, in_dim))).astype(np.float16).view(np.uint16)
    y = torch.full((B, out_dim), float("nan"), device="cuda")
    hip.proj_f16_x16_fused(y, x16, dev(w))
    check_projection(orc, x, w, host(y).astype(np.float64))
    r0 = rng.standard_normal((B, out_dim)).astype(np.float32)
    y = dev(r0)
    hip.proj_f16_x16_fused(y, x16, dev(w), epilogue=hip.PROJ_ADD)
    ref, mag = _proj_ref(orc, x, w)
    want = r0.astype(np.float64) + ref
    tol = _ulp16(ref) + mag * 2.0 ** -21 * 4 + np.spacing(np.abs(want).astype(np.float32))
    assert np.all(np.abs(host(y).astype(np.float64) - want) <= tol)
    inter = out_dim // 2
    h = torch.full((B, inter), float("nan"), device="cuda")
    hip.proj_f16_x16_fused(h, x16, dev(w[:2 * inter]), epilogue=hip.PROJ_SWIGLU)
    gu, mg = ref[:, :2 * inter], mag[:, :2 * inter]
    g, u, m_g, m_u = gu[:, :inter], gu[:, inter:], mg[:, :inter], mg[:, inter:]
    want = g / (1 + np.exp(-g)) * u
    eg = _ulp16(g) + m_g * 2.0 ** -21 * 4
    eu = _ulp16(u) + m_u * 2.0 ** -21 * 4
    tol = 1.1 * eg * np.abs(u) + np.abs(g / (1 + np.exp(-g))) * eu + eg * eu + np.abs(want) * 1e-6 + 1e-30
    assert np.all(np.abs(host(h).astype(np.float64) - want) <= tol)
    h16 = torch.empty(B, inter, dtype=torch.int16, device="cuda")
    hip.proj_f16_x16_fused(h16, x16, dev(w[:2 * inter]), epilogue=hip.PROJ_SWIGLU_F16)
    assert_bitexact(host(h16), orc.f32_to_f16_rne(host(h)).reshape(B, inter), "fp16 SwiGLU vs fp32 SwiGLU rounded")


def _proj_ref(orc, x, w):
    """The oracle's rounded projection (float64 of fp16 values) and the term
    magnitudes sum |x16| |w| that bound an fp32 accumulation's error."""
    B, in_dim = x.shape
    x16 = orc.f32_to_f16_rne(np.ascontiguousarray(x, np.float32)).reshape(B, in_dim)
    ref = orc.linear_f16(x16, w).view(np.float16).astype(np.float64)
    mag = np.abs(x16.view(np.float16).astype(np.float64)) @ np.abs(w.view(np.float16).astype(np.float64)).T
    return ref, mag


def _ulp16(v):
    return np.spacing(np.abs(v).astype(np.float16)).astype(np.float64)


@pytest.mark.parametrize("B,out_dim,in_dim,same_kernel", [(64, 151936, 1024, True), (20, 70001, 256, True),
                                                           (17, 8192, 4096, True), (1, 8200, 512, False),
                                                           (33, 16, 4096, False), (5, 1000, 256, False)])
def test_proj_tiled(hip, orc, rng, B, out_dim, in_dim, same_kernel):
    """W in the tiled layout (rows past out_dim zero): fp32 and fp16 outputs
    bit-identical to the row-major LDS kernel where anelm_proj_f16_x16_fused
    and anelm_linear_f16 take it (more than 16 rows, at least 8192 output
    rows), and against the oracle everywhere, including a ragged last tile."""
    import torch

    w = (0.03 * rng.standard_normal((out_dim, in_dim))).astype(np.float16).view(np.uint16)
    x = rng.standard_normal((B, in_dim)).astype(np.float32)
    x16 = dev(orc.f32_to_f16_rne(x).reshape(B, in_dim).view(np.int16))
    dw = dev(w)
    wt = torch.full((hip.proj_tiled_size(out_dim, in_dim) // 2,), -1, dtype=torch.int16, device="cuda")
    hip.proj_tile_f16(wt, dw)
    padded = host(wt).reshape(-1)
    tiles = (out_dim + 15) // 16
    # piece l of (tile t, step s) = W[16t + l % 16][32s + 8(l // 16) .. +7]
    want_layout = np.zeros((tiles * 16, in_dim), np.uint16)
    want_layout[:out_dim] = w
    want_layout = want_layout.reshape(tiles, 16, in_dim // 32, 4, 8).transpose(0, 2, 3, 1, 4).reshape(-1)
    assert np.array_equal(padded.view(np.uint16), want_layout)
    y = torch.full((B, out_dim), float("nan"), device="cuda")
    hip.proj_f16_x16_tiled(y, x16, wt, out_dim)
    y16 = torch.empty(B, out_dim, dtype=torch.int16, device="cuda")
    hip.proj_f16_x16_tiled(y16, x16, wt, out_dim, epilogue=hip.PROJ_STORE_F16)
    assert_bitexact(host(y16).view(np.float16).astype(np.float32), host(y), "fp16 output = fp32 output narrowed")
    if same_kernel:
        yr = torch.empty(B, out_dim, device="cuda")
        hip.proj_f16_x16_fused(yr, x16, dw)
        assert_bitexact(host(y), host(yr), "tiled vs row-major")
        yr16 = torch.empty(B, out_dim, dtype=torch.int16, device="cuda")
        hip.linear_f16(yr16, x16, dw)
        assert_bitexact(host(y16), host(yr16), "tiled vs row-major, fp16 out")
    check_projection(orc, x, w, host(y).astype(np.float64))


@pytest.mark.parametrize("B,out_dim,in_dim", [(64, 4096, 1024), (64, 1024, 2048), (64, 1024, 3072), (17, 1000, 256),
                                               (40, 3072, 1024), (33, 784, 96), (20, 6144, 1024), (64, 16, 4096)])
def test_proj_tiled_epilogues(hip, orc, rng, B, out_dim, in_dim):
    """Past 16 rows the tiled W gives every epilogue the same bits as the
    row-major W (the same kernels on the same operands): store, residual add,
    SwiGLU in fp32 and fp16, and the fp16 store is the fp32 store narrowed."""
    import torch

    x16 = dev(orc.f32_to_f16_rne((2 * rng.standard_normal((B, in_dim))).astype(np.float32)).reshape(B, in_dim)
              .view(np.int16))
    w = (0.03 * rng.standard_normal((out_dim, in_dim))).astype(np.float16).view(np.uint16)
    dw = dev(w)
    wt = torch.full((hip.proj_tiled_size(out_dim, in_dim) // 2,), -1, dtype=torch.int16, device="cuda")
    hip.proj_tile_f16(wt, dw)
    r0 = rng.standard_normal((B, out_dim)).astype(np.float32)
    for epi in (hip.PROJ_STORE, hip.PROJ_ADD):
        yt, yr = dev(r0), dev(r0)
        hip.proj_f16_x16_tiled(yt, x16, wt, out_dim, epilogue=epi)
        hip.proj_f16_x16_fused(yr, x16, dw, epilogue=epi)
        assert_bitexact(host(yt), host(yr), f"tiled vs row-major, epilogue {epi}")
    y16 = torch.empty(B, out_dim, dtype=torch.int16, device="cuda")
    hip.proj_f16_x16_tiled(y16, x16, wt, out_dim, epilogue=hip.PROJ_STORE_F16)
    ys = torch.empty(B, out_dim, device="cuda")
    hip.proj_f16_x16_tiled(ys, x16, wt, out_dim)
    assert_bitexact(host(y16), orc.f32_to_f16_rne(host(ys)).reshape(B, out_dim), "fp16 store = fp32 store narrowed")
    if out_dim % 32 == 0:   # the SwiGLU: out_dim/2 gate rows (a multiple of 16), then the up rows
        inter = out_dim // 2
        for epi, dt in ((hip.PROJ_SWIGLU, torch.float32), (hip.PROJ_SWIGLU_F16, torch.int16)):
            ht = torch.full((B, inter), -1, dtype=dt, device="cuda")
            hr = torch.full((B, inter), -1, dtype=dt, device="cuda")
            hip.proj_f16_x16_tiled(ht, x16, wt, inter, epilogue=epi)
            hip.proj_f16_x16_fused(hr, x16, dw, epilogue=epi)
            assert_bitexact(host(ht), host(hr), f"tiled vs row-major SwiGLU, epilogue {epi}")


@pytest.mark.parametrize("B,out_dim,in_dim", [(1, 1024, 1024), (11, 4096, 1024), (16, 300, 256), (3, 151936, 1024),
                                               (1, 4097, 1024), (2, 4101, 992), (1, 32771, 512), (1, 151936, 1024),
                                               (4, 777, 3072), (1, 1024, 4096), (2, 512, 5120), (8, 1024, 2048)])
def test_proj_fused_rmsnorm_prologue(hip, orc, rng, B, out_dim, in_dim):
    """The fused RMSNorm equals the oracle's RMSNorm followed by the
    projection (the normalised row rounded to fp16 on the way in)."""
    import torch

    x = (2 * rng.standard_normal((B, in_dim))).astype(np.float32)
    gamma = bf16(1 + 0.1 * rng.standard_normal(in_dim))
    w = (0.03 * rng.standard_normal((out_dim, in_dim))).astype(np.float16).view(np.uint16)
    y = torch.full((B, out_dim), float("nan"), device="cuda")
    hip.proj_f16_fused(y, dev(x), dev(w), norm=dev(gamma.view(np.int16)), eps=1e-6)
    xn = np.stack([orc.rmsnorm(x[b], from_bf16(gamma), 1e-6) for b in range(B)])
    check_projection(orc, xn, w, host(y).astype(np.float64))


@pytest.mark.parametrize("B,out_dim,in_dim", [(1, 1024, 2048), (7, 1024, 3072), (16, 256, 512), (2, 1023, 4096),
                                               (1, 1024, 3072), (8, 1000, 992)])
def test_proj_fused_residual_add(hip, orc, rng, B, out_dim, in_dim):
    import torch

    x = rng.standard_normal((B, in_dim)).astype(np.float32)
    w = (0.03 * rng.standard_normal((out_dim, in_dim))).astype(np.float16).view(np.uint16)
    r0 = rng.standard_normal((B, out_dim)).astype(np.float32)
    y = dev(r0)
    hip.proj_f16_fused(y, dev(x), dev(w), epilogue=hip.PROJ_ADD)
    ref, mag = _proj_ref(orc, x, w)
    want = r0.astype(np.float64) + ref
    got = host(y).astype(np.float64)
    tol = _ulp16(ref) + mag * 2.0 ** -21 * 4 + np.spacing(np.abs(want).astype(np.float32))
    assert np.all(np.abs(got - want) <= tol)


@pytest.mark.parametrize("B,inter,in_dim,norm", [(1, 3072, 1024, True), (5, 384, 256, True), (16, 160, 64, False),
                                                   (2, 3072, 1024, True), (1, 1001, 4096, False), (8, 512, 1024, True)])
def test_proj_fused_swiglu(hip, orc, rng, B, inter, in_dim, norm):
    """gate|up projection with the SwiGLU epilogue: silu(g) * u of the rounded
    gate and up projections, in the fp32 form of core/cpu_ops.cpp:7-14."""
    import torch

    x = (2 * rng.standard_normal((B, in_dim))).astype(np.float32)
    gamma = bf16(1 + 0.1 * rng.standard_normal(in_dim))
    w = (0.05 * rng.standard_normal((2 * inter, in_dim))).astype(np.float16).view(np.uint16)
    h = torch.full((B, inter), float("nan"), device="cuda")
    hip.proj_f16_fused(h, dev(x), dev(w), norm=dev(gamma.view(np.int16)) if norm else None, eps=1e-6,
                       epilogue=hip.PROJ_SWIGLU)
    xn = np.stack([orc.rmsnorm(x[b], from_bf16(gamma), 1e-6) for b in range(B)]) if norm else x
    gu, mag = _proj_ref(orc, xn, w)
    g, u, mg, mu = gu[:, :inter], gu[:, inter:], mag[:, :inter], mag[:, inter:]
    want = g / (1 + np.exp(-g)) * u
    # each rounded projection may be off by its tolerance; silu' <= 1.1
    eg = _ulp16(g) + mg * 2.0 ** -21 * 4
    eu = _ulp16(u) + mu * 2.0 ** -21 * 4
    tol = 1.1 * eg * np.abs(u) + np.abs(g / (1 + np.exp(-g))) * eu + eg * eu + np.abs(want) * 1e-6 + 1e-30
    assert np.all(np.abs(host(h).astype(np.float64) - want) <= tol)


@pytest.mark.parametrize("B,inter,in_dim,norm", [(1, 3072, 1024, True), (2, 3072, 1024, False), (1, 1001, 4096, True),
                                                   (16, 384, 256, True), (40, 512, 1024, False), (5, 160, 5120, True)])
def test_proj_fused_swiglu_f16(hip, orc, rng, B, inter, in_dim, norm):
    """The fp32-input SwiGLU stored as fp16 (the down projection's input)
    is the fp32 SwiGLU rounded to nearest even, bit for bit, on the dot and
    MFMA paths, with and without the fused RMSNorm."""
    import torch

    x = (2 * rng.standard_normal((B, in_dim))).astype(np.float32)
    gamma = dev(bf16(1 + 0.1 * rng.standard_normal(in_dim)).view(np.int16)) if norm else None
    w = dev((0.05 * rng.standard_normal((2 * inter, in_dim))).astype(np.float16).view(np.uint16))
    h = torch.full((B, inter), float("nan"), device="cuda")
    hip.proj_f16_fused(h, dev(x), w, norm=gamma, eps=1e-6, epilogue=hip.PROJ_SWIGLU)
    h16 = torch.full((B, inter), -1, dtype=torch.int16, device="cuda")
    hip.proj_f16_fused(h16, dev(x), w, norm=gamma, eps=1e-6, epilogue=hip.PROJ_SWIGLU_F16)
    assert_bitexact(host(h16), orc.f32_to_f16_rne(host(h)).reshape(B, inter), "fp16 SwiGLU vs fp32 SwiGLU rounded")


@pytest.mark.parametrize("B,out_dim,in_dim", [(1, 1024, 2048), (1, 1024, 3072), (2, 1024, 3072), (1, 4096, 1024),
                                               (2, 6000, 1024), (1, 151936, 1024), (4, 1024, 1024), (8, 640, 4096)])
def test_proj_x16_matches_f32_rows(hip, orc, rng, B, out_dim, in_dim):
    """Rows that are exact fp16 values give the same bits through the fp32
    entry (rounded per element in the kernel) and the fp16 entry (rounded by
    their producer): the decode step hands the o and down projections fp16
    rows on that basis."""
    import torch

    x16 = orc.f32_to_f16_rne((2 * rng.standard_normal((B, in_dim))).astype(np.float32)).reshape(B, in_dim)
    x = x16.view(np.float16).astype(np.float32)
    w = dev((0.03 * rng.standard_normal((out_dim, in_dim))).astype(np.float16).view(np.uint16))
    r0 = rng.standard_normal((B, out_dim)).astype(np.float32)
    for epi in (hip.PROJ_STORE, hip.PROJ_ADD):
        y32, y16 = dev(r0), dev(r0)
        hip.proj_f16_fused(y32, dev(x), w, epilogue=epi)
        hip.proj_f16_x16_fused(y16, dev(x16.view(np.int16)), w, epilogue=epi)
        assert_bitexact(host(y16), host(y32), f"x16 vs fp32 rows, epilogue {epi}")


@pytest.mark.parametrize("tied,B", [(True, 3), (False, 3), (True, 11), (True, 1), (True, 20), (False, 33)])
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
    pos0 = np.resize(np.array([0, 100, 20000]), B)    # every third sequence uses the RoPE fallback
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


@pytest.mark.parametrize("B,out_dim,in_dim", [(2, 1024, 2048), (20, 512, 256), (1, 3000, 1024)])
def test_proj_fused_strided_rows(hip, orc, rng, B, out_dim, in_dim):
    """x and y as column slices of wider row-major buffers (row strides
    larger than the rows, offsets inside the rows), for the dot kernel
    (B <= 2) and the MFMA kernel, store and residual add; the columns
    outside the slices stay untouched."""
    import torch

    x = rng.standard_normal((B, in_dim)).astype(np.float32)
    w = (0.03 * rng.standard_normal((out_dim, in_dim))).astype(np.float16).view(np.uint16)
    xb = torch.full((B, in_dim + 40), float("nan"), device="cuda")
    xb[:, 8:8 + in_dim] = dev(x)
    yb = torch.full((B, out_dim + 24), -7.0, device="cuda")
    hip.proj_f16_fused(yb[:, 4:4 + out_dim], xb[:, 8:8 + in_dim], dev(w))
    got = host(yb)
    check_projection(orc, x, w, got[:, 4:4 + out_dim].astype(np.float64))
    assert np.all(got[:, :4] == -7.0) and np.all(got[:, 4 + out_dim:] == -7.0)
    r0 = rng.standard_normal((B, out_dim)).astype(np.float32)
    yb[:, 4:4 + out_dim] = dev(r0)
    hip.proj_f16_fused(yb[:, 4:4 + out_dim], xb[:, 8:8 + in_dim], dev(w), epilogue=hip.PROJ_ADD)
    ref, mag = _proj_ref(orc, x, w)
    want = r0.astype(np.float64) + ref
    tol = _ulp16(ref) + mag * 2.0 ** -21 * 4 + np.spacing(np.abs(want).astype(np.float32))
    got = host(yb)
    assert np.all(np.abs(got[:, 4:4 + out_dim].astype(np.float64) - want) <= tol)
    assert np.all(got[:, :4] == -7.0) and np.all(got[:, 4 + out_dim:] == -7.0)


def _decode_vs_oracle(hip, orc, rng, path, t, d, B, steps, cap=16, ld_pad=0, model=None):
    """`steps` decode steps of B sequences through anelm_qwen3_forward
    against the oracle's step; logits land in a [B, V + ld_pad] buffer whose
    padding columns must stay untouched.  With `model` given, that model
    (loaded with capacity `cap` and at least B sequences) is reset and used
    and left open.  Returns the worst row error relative to the row's logit
    scale."""
    import torch

    cfg = hip.Qwen3Config(d["H"], d["L"], d["nq"], d["nk"], d["D"], d["I"], d["V"], 1e6, 1e-6)
    ocfg = orc.Qwen3Config(d["H"], d["L"], d["nq"], d["nk"], d["D"], d["I"], d["V"], 1e6, 1e-6)
    own = model is None
    if own:
        model = hip.Qwen3Model(path, cfg, max_batch=B, kv_capacity=cap)
    else:
        model.reset()
    ref = orc.Qwen3(ocfg, t, B, cap)
    V = d["V"]
    buf = torch.full((B, V + ld_pad), -3.0, device="cuda")
    logits = buf[:, :V]
    pos0 = np.resize(np.array([0, 100, 20000]), B)    # every third sequence uses the RoPE fallback
    worst = 0.0
    for s in range(steps):
        ids = rng.integers(0, V, B).astype(np.int32)
        pos = (pos0 + s).astype(np.int32)
        model.forward(dev(ids), dev(pos), logits)
        want = ref.forward(ids, pos)
        got = host(buf)
        assert np.all(got[:, V:] == -3.0), "logits padding written"
        err = np.max(np.abs(got[:, :V] - want), axis=1) / np.max(np.abs(want), axis=1)
        worst = max(worst, float(err.max()))
    if own:
        model.close()
    return worst


@pytest.mark.parametrize("B,ld_pad", [(17, 0), (20, 0), (20, 40)])
def test_decode_big_vocab_past_16_rows(hip, orc, rng, tmp_path, B, ld_pad):
    """The LM-head branch that Qwen3's 151936-row vocabulary takes with more
    than 16 sequences (vocab above 65536), with the logits rows contiguous
    (ld_logits == V) and strided (ld_logits > V); the rings wrap."""
    t, d = tiny_qwen3(rng, V=70000, tied=False)
    path = tmp_path / "bigvocab.safetensors"
    save_qwen3(path, t)
    assert _decode_vs_oracle(hip, orc, rng, path, t, d, B, steps=18, cap=16, ld_pad=ld_pad) < 4e-3


@pytest.mark.parametrize("B,steps", [(1, 200), (3, 170), (20, 170)])
def test_decode_long_rings_match_oracle(hip, orc, rng, tmp_path, B, steps):
    """Rings longer than one attention chunk: at capacity 160 the rings pass
    128 rows (from then on the attention splits each over 3 chunks of 64,
    and the last chunk to finish merges the partials in-kernel), fill up and
    wrap.  Every step against the oracle."""
    t, d = tiny_qwen3(rng)
    path = tmp_path / "long.safetensors"
    save_qwen3(path, t)
    assert _decode_vs_oracle(hip, orc, rng, path, t, d, B, steps=steps, cap=160) < 4e-3


@pytest.mark.parametrize("B", [3, 9, 20])
def test_decode_dims_not_multiples_of_32(hip, orc, rng, tmp_path, B):
    """Hidden and intermediate sizes that are not multiples of 32 (H 224 is,
    I 336 is not): the decode step's per-op branch, whose projections with
    336 inputs cannot take 32-input MFMA steps whole."""
    t, d = tiny_qwen3(rng, H=224, I=336, V=500, tied=True)
    path = tmp_path / "odd.safetensors"
    save_qwen3(path, t)
    assert _decode_vs_oracle(hip, orc, rng, path, t, d, B, steps=18, cap=16, ld_pad=8) < 4e-3


def test_decode_workspace_reuse_across_batches(hip, orc, rng, tmp_path):
    """One model, so one attention workspace, sized for 64 sequences: 140
    steps of 64 sequences (the rings pass 128 rows and split into chunks
    from then on), then after a reset 140 steps of one sequence and 135 of
    three, each phase against a fresh oracle.  A batch change moves the
    chunking and the partials; the chunk counters must stay where every call
    finds them zeroed."""
    t, d = tiny_qwen3(rng)
    path = tmp_path / "reuse.safetensors"
    save_qwen3(path, t)
    cfg = hip.Qwen3Config(d["H"], d["L"], d["nq"], d["nk"], d["D"], d["I"], d["V"], 1e6, 1e-6)
    model = hip.Qwen3Model(path, cfg, max_batch=64, kv_capacity=160)
    try:
        for B, steps in ((64, 140), (1, 140), (3, 135)):
            assert _decode_vs_oracle(hip, orc, rng, path, t, d, B, steps, cap=160, model=model) < 4e-3, B
    finally:
        model.close()
