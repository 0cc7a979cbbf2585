"""Pins the oracle's one-call layer chain (models/llm/qwen3.cpp:502-528):
orc_layer_chain must equal the composition of the oracle's separately
pinned ops -- RMSNorm, per-head q/k RMSNorm + RoPE, residual add, RMSNorm,
SwiGLU, residual add -- bit for bit, at a Qwen3-0.6B row shape and a small
ragged one, with positions inside and past the RoPE table."""
import numpy as np
import pytest

THETA, EPS, D = 1e6, 1e-6, 128


@pytest.mark.parametrize("T,H,nq,nk,I", [(6, 1024, 16, 8, 3072), (5, 260, 4, 2, 388)])
def test_layer_chain_is_composition_of_pinned_ops(orc, rng, T, H, nq, nk, I):
    rn = lambda *s: rng.standard_normal(s).astype(np.float32)
    x, attn, mlp, q, k, g, u = rn(T, H), rn(T, H), rn(T, H), rn(T, nq * D), rn(T, nk * D), rn(T, I), rn(T, I)
    w_in, w_post = (1 + 0.02 * rn(H)).astype(np.float32), (1 + 0.02 * rn(H)).astype(np.float32)
    wq, wk = (1 + 0.02 * rn(D)).astype(np.float32), (1 + 0.02 * rn(D)).astype(np.float32)
    cos_tab, sin_tab = orc.rope_table(16384, D, THETA)
    pos = rng.integers(0, 40000, T).astype(np.int32)
    pos[0], pos[1] = 0, 16383                      # first and last table rows; the rest mostly past the table

    # the chain, in place
    xc, qc, kc = x.copy(), q.copy(), k.copy()
    xn, h = np.empty((T, H), np.float32), np.empty((T, I), np.float32)
    orc.layer_chain(T, H, nq, nk, D, I, xc, xn, attn, mlp, qc, kc, g, u, h, w_in, w_post, wq, wk, pos, cos_tab,
                    sin_tab, THETA, EPS)

    # the separately pinned ops, in the chain's order
    xn_in = orc.rmsnorm_rows(x, w_in, EPS)                                             # :503
    q2, k2 = orc.qknorm_rope(q, k, wq, wk, pos, cos_tab, sin_tab, THETA, nq, nk, D, EPS)  # :444-472
    x1 = orc.residual_add(x, attn)                                                     # :516
    xn_post = orc.rmsnorm_rows(x1, w_post, EPS)                                        # :518
    h2 = orc.silu_mul(g, u)                                                            # fused_ffn's SwiGLU
    x2 = orc.residual_add(x1, mlp)                                                     # :527

    for name, got, want in (("x", xc, x2), ("xn (post-attention norm)", xn, xn_post), ("q", qc, q2), ("k", kc, k2),
                            ("h", h, h2)):
        assert np.array_equal(got.view(np.uint32), want.view(np.uint32)), name
    # the input norm, which the chain's xn buffer holds only until the
    # post-attention norm overwrites it: one row through the chain alone
    # with attn = 0 and mlp = 0 gives rmsnorm(x) as its post norm with w_post = w_in
    x0, z = x[:1].copy(), np.zeros((1, H), np.float32)
    xn0, h0 = np.empty((1, H), np.float32), np.empty((1, I), np.float32)
    orc.layer_chain(1, H, nq, nk, D, I, x0, xn0, z, z, q[:1].copy(), k[:1].copy(), g[:1], u[:1], h0, w_in, w_in, wq,
                    wk, pos[:1], cos_tab, sin_tab, THETA, EPS)
    assert np.array_equal(xn0.view(np.uint32), xn_in[:1].view(np.uint32))
