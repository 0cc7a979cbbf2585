"""Qwen3.5 linear-attention ops and matvec on the GPU against the oracle
(core/cpu_ops.cpp:33-39, :100-171) at the Qwen3.5-0.8B shapes
(16 key and 16 value heads of 128, conv kernel 4 over 6144 channels,
hidden 1024).  conv1d_update is bit-exact (same fused multiply-adds in the
same order); the others are within 1e-5 relative, measured against the
magnitude of the terms each output sums where outputs can cancel."""
import numpy as np
import pytest

from helpers import REL_TOL, assert_bitexact, dev, host, max_rel_err

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("rows,dim,wdt", [(16, 128, "f32"), (64 * 16, 128, "f16"), (3, 1000, "bf16"), (1, 64, "f32")])
def test_rmsnorm_gated(hip, orc, rng, rows, dim, wdt):
    import torch

    x = rng.standard_normal((rows, dim)).astype(np.float32)
    z = (2 * rng.standard_normal((rows, dim))).astype(np.float32)
    w32 = (1 + 0.1 * rng.standard_normal(dim)).astype(np.float32)
    tw = {"f32": torch.from_numpy(w32), "f16": torch.from_numpy(w32).half(),
          "bf16": torch.from_numpy(w32).bfloat16()}[wdt].cuda()
    wref = tw.float().cpu().numpy()
    out = torch.empty(rows, dim, device="cuda")
    hip.rmsnorm_gated(out, dev(x), dev(z), tw)
    ref = np.stack([orc.rmsnorm_gated(x[r], z[r], wref) for r in range(rows)])
    assert max_rel_err(host(out), ref) <= REL_TOL


def test_rmsnorm_gated_in_place(hip, orc, rng):
    x = rng.standard_normal((32, 128)).astype(np.float32)
    z = rng.standard_normal((32, 128)).astype(np.float32)
    w = np.ones(128, np.float32)
    t = dev(x)
    hip.rmsnorm_gated(t, t, dev(z), dev(w))
    ref = np.stack([orc.rmsnorm_gated(x[r], z[r], w) for r in range(32)])
    assert max_rel_err(host(t), ref) <= REL_TOL


@pytest.mark.parametrize("rows,dim,scale", [(32, 128, 1.0), (64 * 16, 128, float(np.float32(1 / np.sqrt(128)))),
                                            (5, 77, 1.0)])
def test_l2_normalize(hip, orc, rng, rows, dim, scale):
    x = rng.standard_normal((rows, dim)).astype(np.float32)
    x[0] = 0.0                                                     # zero row stays zero
    t = dev(x)
    hip.l2_normalize(t, scale)
    ref = np.stack([orc.l2_normalize(x[r]) * np.float32(scale) for r in range(rows)])
    assert max_rel_err(host(t), ref) <= REL_TOL
    assert np.array_equal(host(t)[0], np.zeros(dim, np.float32))


@pytest.mark.parametrize("B,ch,K", [(1, 6144, 4), (3, 6144, 4), (2, 1000, 3), (64, 6144, 4), (2, 33, 7)])
def test_conv1d_update_bitexact(hip, orc, rng, B, ch, K):
    import torch

    w = rng.standard_normal((ch, K)).astype(np.float32)
    state = rng.standard_normal((B, ch, K - 1)).astype(np.float32)
    pos = (np.arange(B) % (K - 1)).astype(np.int32)
    ds, dp, dw = dev(state), dev(pos), dev(w)
    y = torch.empty(B, ch, device="cuda")
    for step in range(5):
        x = rng.standard_normal((B, ch)).astype(np.float32)
        hip.conv1d_update(y, ds, dp, dev(x), dw)
        got = host(y)
        for b in range(B):
            pb = pos[b:b + 1].copy()
            ref = orc.conv1d_update(state[b], pb, x[b], w)
            pos[b] = pb[0]
            assert_bitexact(got[b], ref, f"y step {step} seq {b}")
        assert np.array_equal(host(dp), pos)
    assert_bitexact(host(ds), state, "conv state")


@pytest.mark.parametrize("B,nvh,nkh,kd,vd", [(1, 16, 16, 128, 128), (4, 16, 16, 128, 128), (2, 16, 8, 128, 128),
                                             (3, 4, 2, 64, 64), (2, 2, 1, 256, 128), (1, 3, 3, 256, 64)])
def test_ssm_step(hip, orc, rng, B, nvh, nkh, kd, vd):
    import torch

    S = (0.1 * rng.standard_normal((B, nvh, kd, vd))).astype(np.float32)
    q = rng.standard_normal((B, nkh * kd)).astype(np.float32)
    k = rng.standard_normal((B, nkh * kd)).astype(np.float32)
    k /= np.linalg.norm(k.reshape(B, nkh, kd), axis=2).repeat(kd, axis=1).astype(np.float32)
    v = rng.standard_normal((B, nvh * vd)).astype(np.float32)
    decay = rng.uniform(0.5, 1.0, (B, nvh)).astype(np.float32)
    beta = rng.uniform(0.0, 1.0, (B, nvh)).astype(np.float32)
    dS = dev(S)
    y = torch.empty(B, nvh * vd, device="cuda")
    hip.ssm_step(y, dS, dev(q), dev(k), dev(v), dev(decay), dev(beta), nkh)
    gS, gy = host(dS), host(y).reshape(B, nvh, vd)
    per = nvh // nkh
    for b in range(B):
        for h in range(nvh):
            kh = h // per
            st = S[b, h].copy()
            qh, khv = q[b, kh * kd:(kh + 1) * kd], k[b, kh * kd:(kh + 1) * kd]
            yref = orc.ssm_step(st, qh, khv, v[b, h * vd:(h + 1) * vd], decay[b, h], beta[b, h])
            Sd = S[b, h].astype(np.float64)
            delta = v[b, h * vd:(h + 1) * vd] - Sd.T @ khv
            scale = np.abs(decay[b, h] * Sd) + np.abs(beta[b, h] * np.outer(khv, delta))
            assert np.max(np.abs(gS[b, h] - st) / (scale + 1e-30)) <= REL_TOL
            ybound = np.abs(st.astype(np.float64)).T @ np.abs(qh)
            assert np.max(np.abs(gy[b, h] - yref) / (ybound + 1e-30)) <= REL_TOL


@pytest.mark.parametrize("out_dim,in_dim", [(16, 1024), (151936, 1024), (1000, 1001), (7, 4)])
def test_matvec(hip, orc, rng, out_dim, in_dim):
    import torch

    W = rng.standard_normal((out_dim, in_dim)).astype(np.float32)
    x = rng.standard_normal(in_dim).astype(np.float32)
    y = torch.empty(out_dim, device="cuda")
    hip.matvec(y, dev(W), dev(x))
    ref = orc.matvec(W, x)
    bound = np.abs(W).astype(np.float64) @ np.abs(x)
    assert np.max(np.abs(host(y) - ref) / bound) <= REL_TOL


def test_head_slices_of_fused_rows(hip, orc, rng):
    """The batched layer's layout: q, k are head slices of the fused conv
    output row and z a slice of the projection row (qwen3_5.cpp:503-549)."""
    import torch

    B, nkh, nvh, kd, vd = 5, 16, 16, 128, 128
    ch = 2 * nkh * kd + nvh * vd
    mixed = rng.standard_normal((B, ch)).astype(np.float32)
    t = dev(mixed)
    qs = float(np.float32(1 / np.sqrt(kd)))
    hip.l2_normalize(t[:, :nkh * kd], qs, heads=nkh)
    hip.l2_normalize(t[:, nkh * kd:2 * nkh * kd], 1.0, heads=nkh)
    got = host(t)
    ref = mixed.copy()
    for b in range(B):
        for h in range(2 * nkh):
            ref[b, h * kd:(h + 1) * kd] = orc.l2_normalize(mixed[b, h * kd:(h + 1) * kd]) * (np.float32(qs) if h < nkh else 1)
    assert max_rel_err(got, ref) <= REL_TOL
    qkvz = rng.standard_normal((B, ch + nvh * vd)).astype(np.float32)
    y = rng.standard_normal((B, nvh * vd)).astype(np.float32)
    w = (1 + 0.05 * rng.standard_normal(vd)).astype(np.float32)
    dz = dev(qkvz)
    out = torch.empty(B, nvh * vd, device="cuda")
    hip.rmsnorm_gated(out, dev(y), dz[:, ch:], dev(w), heads=nvh)
    z = qkvz[:, ch:]
    ref = np.stack([np.concatenate([orc.rmsnorm_gated(y[b, h * vd:(h + 1) * vd], z[b, h * vd:(h + 1) * vd], w)
                                    for h in range(nvh)]) for b in range(B)])
    assert max_rel_err(host(out), ref) <= REL_TOL


# 128-channel blocks per sequence: 48 (3 per wave of 16), 8 and 3 (one each),
# 24 (2 per wave), 56 (4 per wave) and 104 (two passes of up to 4 per wave)
@pytest.mark.parametrize("B,nkh,nvh,steps", [(1, 16, 16, 5), (64, 16, 16, 4), (3, 2, 4, 7), (2, 0, 3, 2),
                                             (2, 8, 8, 3), (3, 16, 24, 3), (2, 32, 40, 4)])
def test_conv_silu_l2norm_matches_separate_calls(hip, rng, B, nkh, nvh, steps):
    """The fused conv1d update + SiLU + q/k L2 norm equals anelm_conv1d_update,
    anelm_silu and two anelm_l2_normalize calls bit for bit (outputs, ring
    states and positions), over several steps so the ring wraps."""
    import torch

    ch = (2 * nkh + nvh) * 128
    qs = float(1.0 / np.sqrt(128.0))
    w = dev((0.5 * rng.standard_normal((ch, 4))).astype(np.float32))
    st0 = rng.standard_normal((B, ch, 3)).astype(np.float32)
    pos0 = rng.integers(-1, 4, B).astype(np.int32)        # out-of-range positions are taken as 0
    sa, pa, sb, pb = dev(st0), dev(pos0), dev(st0), dev(pos0)
    for _ in range(steps):
        x = dev((2 * rng.standard_normal((B, ch))).astype(np.float32))
        ya = torch.empty(B, ch, device="cuda")
        hip.conv1d_update(ya, sa, pa, x, w)
        hip.silu(ya)
        if nkh:
            hip.l2_normalize(ya[:, :nkh * 128], qs, heads=nkh)
            hip.l2_normalize(ya[:, nkh * 128:2 * nkh * 128], 1.0, heads=nkh)
        yb = torch.empty(B, ch, device="cuda")
        hip.conv1d_silu_l2norm(yb, sb, pb, x, w, nkh, qs)
        assert_bitexact(host(yb), host(ya), "outputs")
        assert_bitexact(host(sb), host(sa), "conv states")
        assert np.array_equal(host(pb), host(pa))


@pytest.mark.parametrize("B,nvh,nkh,kd,vd,wdt", [(64, 16, 16, 128, 128, "f32"), (1, 16, 16, 128, 128, "bf16"),
                                                 (3, 8, 2, 64, 64, "f16"), (2, 4, 4, 256, 128, "f32")])
def test_ssm_step_gated_norm_matches_separate_calls(hip, rng, B, nvh, nkh, kd, vd, wdt):
    """The state step with the gated RMSNorm fused in equals anelm_ssm_step
    then anelm_rmsnorm_gated bit for bit (outputs and states)."""
    import torch

    S0 = (0.05 * rng.standard_normal((B, nvh, kd, vd))).astype(np.float32)
    q = dev(rng.standard_normal((B, nkh * kd)).astype(np.float32))
    k = dev(rng.standard_normal((B, nkh * kd)).astype(np.float32))
    v = dev(rng.standard_normal((B, nvh * vd)).astype(np.float32))
    z = dev((2 * rng.standard_normal((B, nvh * vd))).astype(np.float32))
    decay = dev(rng.uniform(0.5, 1.0, (B, nvh)).astype(np.float32))
    beta = dev(rng.uniform(0.0, 1.0, (B, nvh)).astype(np.float32))
    w32 = (1 + 0.1 * rng.standard_normal(vd)).astype(np.float32)
    nw = {"f32": torch.from_numpy(w32), "f16": torch.from_numpy(w32).half(),
          "bf16": torch.from_numpy(w32).bfloat16()}[wdt].cuda()
    Sa, Sb = dev(S0), dev(S0)
    y = torch.empty(B, nvh * vd, device="cuda")
    outa = torch.empty(B, nvh * vd, device="cuda")
    hip.ssm_step(y, Sa, q, k, v, decay, beta, nkh)
    hip.rmsnorm_gated(outa, y, z, nw, heads=nvh)
    outb = torch.full((B, nvh * vd), float("nan"), device="cuda")
    hip.ssm_step_gated_norm(outb, Sb, q, k, v, decay, beta, z, nw, nkh)
    assert_bitexact(host(outb), host(outa), "gated outputs")
    assert_bitexact(host(Sb), host(Sa), "states")


@pytest.mark.parametrize("B,nh,wdt,steps,pad", [(64, 16, "f32", 4, 0), (1, 16, "bf16", 5, 0), (3, 2, "f16", 4, 128),
                                                (5, 3, "f32", 3, 0)])
def test_conv_ssm_step_gated_norm_matches_two_calls(hip, rng, B, nh, wdt, steps, pad):
    """The one-launch conv + SiLU + L2 norm + state step + gated RMSNorm equals
    anelm_conv1d_silu_l2norm then anelm_ssm_step_gated_norm bit for bit
    (outputs, delta-rule states, conv rings, ring positions), over several
    steps so the ring wraps; x and z as views into wider rows when pad > 0."""
    import torch

    ch, n = 3 * nh * 128, nh * 128
    qs = float(1.0 / np.sqrt(128.0))
    cw = dev((0.5 * rng.standard_normal((ch, 4))).astype(np.float32))
    ring0 = rng.standard_normal((B, ch, 3)).astype(np.float32)
    S0 = (0.05 * rng.standard_normal((B, nh, 128, 128))).astype(np.float32)
    pos0 = rng.integers(-1, 4, B).astype(np.int32)          # out-of-range positions are taken as 0
    w32 = (1 + 0.1 * rng.standard_normal(128)).astype(np.float32)
    nw = {"f32": torch.from_numpy(w32), "f16": torch.from_numpy(w32).half(),
          "bf16": torch.from_numpy(w32).bfloat16()}[wdt].cuda()
    Sa, ra, pa = dev(S0), dev(ring0), dev(pos0)
    Sb, rb, pb = dev(S0), dev(ring0), dev(np.repeat(pos0, nh))
    mixed = torch.empty(B, ch, device="cuda")
    for step in range(steps):
        xz = dev((2 * rng.standard_normal((B, ch + n + pad))).astype(np.float32))
        x, z = xz[:, :ch], xz[:, ch + pad:]
        decay = dev(rng.uniform(0.5, 1.0, (B, nh)).astype(np.float32))
        beta = dev(rng.uniform(0.0, 1.0, (B, nh)).astype(np.float32))
        outa = torch.empty(B, n, device="cuda")
        hip.conv1d_silu_l2norm(mixed, ra, pa, x, cw, nh, qs)
        hip.ssm_step_gated_norm(outa, Sa, mixed[:, :n], mixed[:, n:2 * n], mixed[:, 2 * n:], decay, beta, z, nw, nh)
        outb = torch.full((B, n), float("nan"), device="cuda")
        hip.conv_ssm_step_gated_norm(outb, Sb, rb, pb, x, cw, decay, beta, z, nw, qs)
        assert_bitexact(host(outb), host(outa), f"step {step}: gated outputs")
        assert_bitexact(host(Sb), host(Sa), f"step {step}: states")
        assert_bitexact(host(rb), host(ra), f"step {step}: conv rings")
        assert np.array_equal(host(pb).reshape(B, nh), np.repeat(host(pa)[:, None], nh, axis=1)), f"step {step}"
