"""anelm_layer_ops (a layer's five ops in one launch) against the five
separate launches it replaces, bit for bit, over several layers at the
decode and prefill-row shapes and at the two full prefill shapes (0.6B at
2048 tokens: one-wave rows, four to a block; 8B at 8192 tokens: two float4
per lane at 512 lanes; fp16 gammas), and the residual stream against the
oracle's per-token layer chain (models/llm/qwen3.cpp:502-528) on every row;
the norm and SwiGLU outputs against the oracle within 1e-5 (every 64th row
at the full prefill shapes)."""
import numpy as np
import pytest

from helpers import REL_TOL, assert_bitexact, dev, gamma_f16, host, max_rel_err

pytestmark = pytest.mark.gpu
THETA, EPS, D = 1e6, 1e-6, 128


@pytest.mark.parametrize("cfg", [
    dict(name="0.6B decode", T=1, H=1024, nq=16, nk=8, I=3072, pmax=4096, layers=28, wdt="f16"),
    dict(name="4B batched decode", T=64, H=2560, nq=32, nk=8, I=9728, pmax=32768, layers=3, wdt="f16"),
    dict(name="0.6B prefill rows", T=64, H=1024, nq=16, nk=8, I=3072, pmax=2048, layers=2, wdt="bf16"),
    dict(name="8B prefill rows", T=16, H=4096, nq=32, nk=8, I=12288, pmax=8192, layers=2, wdt="f32"),
    dict(name="12+4 heads, ragged rows", T=5, H=2600, nq=12, nk=4, I=1000, pmax=40000, layers=2, wdt="f16"),
    dict(name="0.6B prefill", T=2048, H=1024, nq=16, nk=8, I=3072, pmax=2048, layers=2, wdt="f16", geom=(4, 64),
         stride=64),
    dict(name="one-wave rows, ragged block", T=258, H=1024, nq=16, nk=8, I=3072, pmax=2048, layers=1, wdt="bf16",
         geom=(4, 64)),
    dict(name="8B prefill", T=8192, H=4096, nq=32, nk=8, I=12288, pmax=8192, layers=1, wdt="f16", geom=(2, 512),
         stride=64),
], ids=lambda c: c["name"])
def test_layer_ops_equals_five_launches(hip, orc, rng, cfg):
    import torch

    T, H, nq, nk, I = cfg["T"], cfg["H"], cfg["nq"], cfg["nk"], cfg["I"]
    if "geom" in cfg:   # the row geometry the full prefill shapes launch with (fixed by T and H)
        assert hip.rmsnorm_geometry(T, H) == cfg["geom"]
    sel = slice(None, None, cfg.get("stride", 1))
    c_np, s_np = orc.rope_table(16384, D, THETA)
    c_tab, s_tab = dev(c_np), dev(s_np)
    x0 = rng.standard_normal((T, H), dtype=np.float32)
    x_sep, x_one = dev(x0), dev(x0)
    x_ref = x0.copy()

    def gam(n):
        bits = gamma_f16(rng, n)
        if cfg["wdt"] == "f16":
            return dev(bits).view(torch.float16), bits.view(np.float16).astype(np.float32)
        f = bits.view(np.float16).astype(np.float32)
        if cfg["wdt"] == "f32":
            return dev(f), f
        b = (f.view(np.uint32) >> 16).astype(np.uint16)   # bf16 (exact for these values' top bits)
        return dev(b).view(torch.bfloat16), (b.astype(np.uint32) << 16).view(np.float32)

    for layer in range(cfg["layers"]):
        rn = lambda *s: rng.standard_normal(s, dtype=np.float32)
        attn, mlp, q, k, g, u = rn(T, H), rn(T, H), rn(T, nq * D), rn(T, nk * D), rn(T, I), rn(T, I)
        (w_in, w_in32), (w_post, w_post32), (wq, wq32), (wk, wk32) = gam(H), gam(H), gam(D), gam(D)
        pos = rng.integers(0, cfg["pmax"], T).astype(np.int32)
        dpos = dev(pos)
        x_prev = x_ref.copy()
        # the five separate launches
        q1, k1, h1 = dev(q), dev(k), torch.empty(T, I, device="cuda")
        xn_a, xn_b = torch.empty(T, H, device="cuda"), torch.empty(T, H, device="cuda")
        da, dm = dev(attn), dev(mlp)
        hip.rmsnorm(xn_a, x_sep, w_in, EPS)
        hip.qknorm_rope(q1, k1, wq, wk, dpos, c_tab, s_tab, THETA, EPS, nq=nq, nk=nk)
        hip.add_rmsnorm(x_sep, da, xn_b, w_post, EPS)
        hip.silu_mul(h1, dev(g), dev(u))
        hip.residual_add(x_sep, dm)
        # one launch
        q2, k2 = dev(q), dev(k)
        h2 = torch.full((T, I), float("nan"), device="cuda")
        xn_in = torch.full((T, H), float("nan"), device="cuda")
        xn_post = torch.full((T, H), float("nan"), device="cuda")
        hip.layer_ops(x_one, xn_in, xn_post, da, dm, q2, k2, h2, dev(g), dev(u), w_in, w_post, wq, wk, dpos,
                      c_tab, s_tab, THETA, EPS, nq=nq, nk=nk)
        for name, a, b in (("x", x_one, x_sep), ("xn_in", xn_in, xn_a), ("xn_post", xn_post, xn_b), ("q", q2, q1),
                           ("k", k2, k1), ("h", h2, h1)):
            assert_bitexact(host(a), host(b), f"layer {layer}: {name}")
        # the oracle's chain on the same inputs: the residual stream is exact
        xn_r, h_r = np.empty((T, H), np.float32), np.empty((T, I), np.float32)
        qr, kr = q.copy(), k.copy()
        orc.layer_chain(T, H, nq, nk, D, I, x_ref, xn_r, attn, mlp, qr, kr, g, u, h_r, w_in32, w_post32, wq32, wk32,
                        pos, c_np, s_np, THETA, EPS)
        assert_bitexact(host(x_one), x_ref, f"layer {layer}: residual stream vs oracle")
        xn_in_r = np.stack([orc.rmsnorm(r, w_in32, EPS) for r in x_prev[sel]])
        assert max_rel_err(host(xn_in)[sel], xn_in_r) <= REL_TOL
        assert max_rel_err(host(xn_post)[sel], xn_r[sel]) <= REL_TOL
        assert max_rel_err(host(h2)[sel], h_r[sel]) <= REL_TOL


def test_layer_ops_rejects_bad_arguments(hip):
    import torch

    T, H, I = 2, 1024, 3072
    f = lambda *s: torch.zeros(*s, device="cuda")
    args = [f(T, H), f(T, H), f(T, H), f(T, H), f(T, H), f(T, 2048), f(T, 1024), f(T, I), f(T, I), f(T, I),
            f(H).half(), f(H).half(), f(128).half(), f(128).half(), torch.zeros(T, dtype=torch.int32, device="cuda"),
            f(16, 64), f(16, 64)]
    with pytest.raises(hip.AnelmError):   # hidden not a multiple of 4
        hip.layer_ops(f(T, 1022), *args[1:])
    bad = list(args)
    bad[15] = f(0, 64)                    # no RoPE table rows
    with pytest.raises(hip.AnelmError):
        hip.layer_ops(*bad)
