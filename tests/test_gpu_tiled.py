"""The tiled activation path of the decode step past 16 sequences: fp16
rows in the tiled layout of anelm_proj_tile_f16 (16 rows x 32 columns per
contiguous 1 KB piece), written by the RMSNorm, the fused attention and the
SwiGLU, and read by anelm_proj_f16_tt.  Each tiled output, untiled, is
bit-identical to its row-major counterpart, and the tiled projection to the
row-major kernels on the same operands (models/llm/qwen3.cpp:497-528)."""
import numpy as np
import pytest

from helpers import assert_bitexact, bf16, dev, host

pytestmark = pytest.mark.gpu
THETA = 1e6
EPS = 1e-6


def untile(flat, rows, cols):
    """The [rows, cols] matrix of a tiled fp16 buffer (piece l of block (t, s)
    holds row 16t + l%16, columns 32s + 8(l//16) .. +7)."""
    tiles = (rows + 15) // 16
    a = np.asarray(flat).reshape(-1)[:tiles * 16 * cols].reshape(tiles, cols // 32, 4, 16, 8)
    return a.transpose(0, 3, 1, 2, 4).reshape(tiles * 16, cols)[:rows]


def tiled_buf(rows, cols):
    import torch

    return torch.full(((rows + 15) // 16 * 16 * cols,), -1, dtype=torch.int16, device="cuda")


@pytest.mark.parametrize("rows,dim", [(64, 1024), (17, 1024), (33, 4096), (5, 96), (100, 2048)])
def test_rmsnorm_f16_tiled(hip, rng, rows, dim):
    import torch

    x = dev((2 * rng.standard_normal((rows, dim))).astype(np.float32))
    w = dev(bf16(1 + 0.1 * rng.standard_normal(dim)).view(np.int16)).view(torch.bfloat16)
    ref = torch.empty(rows, dim, dtype=torch.int16, device="cuda")
    hip.rmsnorm_f16(ref, x, w, eps=EPS)
    out = tiled_buf(rows, dim)
    hip.rmsnorm_f16_tiled(out, x, w, eps=EPS)
    assert_bitexact(untile(host(out), rows, dim), host(ref), "tiled RMSNorm vs rows")


def test_rmsnorm_f16_tiled_rejects(hip):
    import torch

    x = torch.zeros(4, 100, device="cuda")
    w = torch.ones(100, device="cuda").bfloat16()
    with pytest.raises(Exception):
        hip.rmsnorm_f16_tiled(torch.zeros(16 * 128, dtype=torch.int16, device="cuda"), x, w)   # dim % 32


@pytest.mark.parametrize("B,nq,nk,cap", [(64, 16, 8, 64), (20, 32, 8, 300), (17, 8, 8, 40)])
def test_attention_qk_tiled_output(hip, orc, rng, B, nq, nk, cap):
    """The fused attention's tiled fp16 output equals its fp16 rows, over
    rings of random start and length (long rings merged across chunks)."""
    import torch

    D = 128
    qkv = rng.standard_normal((B, (nq + 2 * nk) * D), dtype=np.float32)
    pos = rng.integers(0, 3000, B).astype(np.int32)
    wq = dev(bf16(1 + 0.1 * rng.standard_normal(D)).view(np.int16)).view(torch.bfloat16)
    wk = dev(bf16(1 + 0.1 * rng.standard_normal(D)).view(np.int16)).view(torch.bfloat16)
    c_tab, s_tab = orc.rope_table(2048, D, THETA)
    kc0 = rng.standard_normal((B, cap, nk * D), dtype=np.float32)
    vc0 = rng.standard_normal((B, cap, nk * D), dtype=np.float32)
    rs0 = rng.integers(0, cap, B).astype(np.int32)
    rl0 = rng.integers(0, cap + 1, B).astype(np.int32)
    rl0[0] = cap
    outs = []
    for tiled in (False, True):
        a = dev(qkv)
        kc, vc, rs, rl = dev(kc0), dev(vc0), dev(rs0), dev(rl0)
        hip.kv_ring_advance(rs, rl, cap)
        ws = torch.zeros(max(hip.gqa_workspace_size(B, nq, nk, D, cap), 16), dtype=torch.uint8, device="cuda")
        out = tiled_buf(B, nq * D) if tiled else torch.full((B, nq * D), -1, dtype=torch.int16, device="cuda")
        hip.gqa_attention_qk(out, a[:, :nq * D], a[:, nq * D:(nq + nk) * D], a[:, (nq + nk) * D:], wq, wk, dev(pos),
                             dev(c_tab), dev(s_tab), kc, vc, rs, rl, nq, nk, ws, THETA, EPS, tiled=tiled)
        outs.append(untile(host(out), B, nq * D) if tiled else host(out))
    assert_bitexact(outs[1], outs[0], "tiled attention output vs rows")


@pytest.mark.parametrize("B,out_dim,in_dim", [(64, 4096, 1024), (64, 1024, 2048), (64, 1024, 3072), (17, 1000, 256),
                                               (40, 3072, 1024), (20, 6144, 1024), (64, 16, 4096), (18, 512, 1024)])
def test_proj_f16_tt(hip, orc, rng, B, out_dim, in_dim):
    """Tiled x and tiled W: every epilogue bit-identical to the tiled-W
    projection on row-major x; the tiled fp16 SwiGLU, untiled, equals the
    fp16 SwiGLU rows."""
    import torch

    x16 = orc.f32_to_f16_rne((2 * rng.standard_normal((B, in_dim))).astype(np.float32)).reshape(B, in_dim)
    xr = dev(x16.view(np.int16))
    xt = tiled_buf(B, in_dim)
    hip.proj_tile_f16(xt, xr)       # the tiled layout of the rows (the W tiling routine, rows = batch rows)
    assert_bitexact(untile(host(xt), B, in_dim), x16.view(np.int16), "tiled x")
    w = dev((0.03 * rng.standard_normal((out_dim, in_dim))).astype(np.float16).view(np.int16))
    wt = torch.full((hip.proj_tiled_size(out_dim, in_dim) // 2,), -1, dtype=torch.int16, device="cuda")
    hip.proj_tile_f16(wt, w)
    r0 = rng.standard_normal((B, out_dim)).astype(np.float32)
    for epi in (hip.PROJ_STORE, hip.PROJ_ADD):
        y, yr = dev(r0), dev(r0)
        hip.proj_f16_tt(y, xt, wt, B, out_dim, in_dim, epilogue=epi)
        hip.proj_f16_x16_tiled(yr, xr, wt, out_dim, epilogue=epi)
        assert_bitexact(host(y), host(yr), f"tiled x vs rows, epilogue {epi}")
    y16 = torch.empty(B, out_dim, dtype=torch.int16, device="cuda")
    yr16 = torch.empty(B, out_dim, dtype=torch.int16, device="cuda")
    hip.proj_f16_tt(y16, xt, wt, B, out_dim, in_dim, epilogue=hip.PROJ_STORE_F16)
    hip.proj_f16_x16_tiled(yr16, xr, wt, out_dim, epilogue=hip.PROJ_STORE_F16)
    assert_bitexact(host(y16), host(yr16), "tiled x vs rows, fp16 store")
    if out_dim % 32 == 0:
        inter = out_dim // 2
        for epi, dt in ((hip.PROJ_SWIGLU, torch.float32), (hip.PROJ_SWIGLU_F16, torch.int16)):
            h = torch.full((B, inter), -1, dtype=dt, device="cuda")
            hr = torch.full((B, inter), -1, dtype=dt, device="cuda")
            hip.proj_f16_tt(h, xt, wt, B, inter, in_dim, epilogue=epi)
            hip.proj_f16_x16_tiled(hr, xr, wt, inter, epilogue=epi)
            assert_bitexact(host(h), host(hr), f"tiled x vs rows, SwiGLU epilogue {epi}")
        if inter % 32 == 0:
            ht = tiled_buf(B, inter)
            hip.proj_f16_tt(ht, xt, wt, B, inter, in_dim, epilogue=hip.PROJ_SWIGLU_F16_TILED)
            assert_bitexact(untile(host(ht), B, inter), host(hr), "tiled fp16 SwiGLU vs rows")


def test_proj_f16_tt_adjacent_buffers(hip, rng):
    """y's 17 rows followed directly by x_t (32 padded rows) in one buffer:
    accepted (the overlap check takes y's own rows, not x_t's padded count),
    and the result equals the same call on separate buffers."""
    import torch

    B, out_dim, in_dim = 17, 64, 256
    buf = torch.zeros(B * out_dim + 32 * in_dim // 2, dtype=torch.float32, device="cuda")
    y = buf[:B * out_dim].view(B, out_dim)
    xt = buf[B * out_dim:].view(torch.int16)
    x16 = (rng.standard_normal((B, in_dim)) * 0.5).astype(np.float16)
    xr = dev(x16.view(np.int16))
    hip.proj_tile_f16(xt, xr)
    w = dev((0.03 * rng.standard_normal((out_dim, in_dim))).astype(np.float16).view(np.int16))
    wt = torch.zeros(hip.proj_tiled_size(out_dim, in_dim) // 2, dtype=torch.int16, device="cuda")
    hip.proj_tile_f16(wt, w)
    hip.proj_f16_tt(y, xt, wt, B, out_dim, in_dim, epilogue=hip.PROJ_STORE)
    ref = torch.zeros(B, out_dim, device="cuda")
    xt2 = tiled_buf(B, in_dim)
    hip.proj_tile_f16(xt2, xr)
    hip.proj_f16_tt(ref, xt2, wt, B, out_dim, in_dim, epilogue=hip.PROJ_STORE)
    assert_bitexact(host(y), host(ref), "adjacent y and x_t")
