"""Pins of the oracle's ANE-contraction pieces and Qwen3 decode step:
the RNE fp16 conversion against numpy's float16 cast, the fp16 projection
against a float64 matmul, and the decode step against an independent
numpy float64 restatement of models/llm/qwen3.cpp:497-564 on a tiny model
(the fp16 rounding points of the projections are the only quantisation)."""
import numpy as np
import pytest

from helpers import from_bf16, tiny_qwen3 as tiny_model


def test_f32_to_f16_rne_matches_numpy(orc, rng):
    bounds = np.arange(0, 0x7C01, dtype=np.uint32).astype(np.uint16).view(np.float16).astype(np.float32)
    mids = np.concatenate([(bounds[:-1].astype(np.float64) + bounds[1:]) / 2]).astype(np.float32)
    vals = np.concatenate([bounds, mids, np.nextafter(mids, np.float32(np.inf)), np.nextafter(mids, np.float32(0)),
                           rng.standard_normal(4000).astype(np.float32) * 100,
                           np.array([65519.99, 65520.0, 65536.0, 1e30, 2 ** -25, 2 ** -25 * 1.0000001, 2 ** -26, 0.0],
                                    np.float32)])
    vals = np.concatenate([vals, -vals])
    got = orc.f32_to_f16_rne(vals)
    with np.errstate(over="ignore"):
        want = vals.astype(np.float16).view(np.uint16)
    assert np.array_equal(got, want)
    nan = orc.f32_to_f16_rne(np.array([np.nan], np.float32))[0]
    assert (nan & 0x7C00) == 0x7C00 and (nan & 0x3FF) != 0


def test_linear_f16_is_rounded_float64_matmul(orc, rng):
    x = rng.standard_normal((3, 200)).astype(np.float16)
    w = (0.05 * rng.standard_normal((70, 200))).astype(np.float16)
    y = orc.linear_f16(x.view(np.uint16), w.view(np.uint16))
    ref = (x.astype(np.float64) @ w.astype(np.float64).T).astype(np.float32).astype(np.float16)
    assert np.array_equal(y, ref.view(np.uint16))


def reference_step(orc, t, d, hist, pos):
    """float64 numpy restatement for one sequence: hist = every token so far
    (the ring holds them all), pos = their positions.  Returns logits."""
    H, L, nq, nk, D, I, V = (d[k] for k in ("H", "L", "nq", "nk", "D", "I", "V"))
    f16 = lambda a: a.astype(np.float32).astype(np.float16).astype(np.float64)      # RNE to fp16
    wf16 = lambda n: orc.bf16_to_f16(t[n]).view(np.float16).astype(np.float64)       # truncating weights

    def proj(x, name_or_w):
        w = name_or_w if isinstance(name_or_w, np.ndarray) else wf16(name_or_w).reshape(-1, x.size)
        return f16(w @ f16(x))

    def rms(x, w):
        return x / np.sqrt(np.mean(x * x) + 1e-6) * w

    theta = 1e6
    inv = 1.0 / theta ** (np.arange(0, D, 2) / D)
    ks = [[None] * len(hist) for _ in range(L)]
    vs = [[None] * len(hist) for _ in range(L)]
    out = None
    for ti, (tok, p) in enumerate(zip(hist, pos)):
        x = from_bf16(t["model.embed_tokens.weight"]).reshape(V, H)[tok].astype(np.float64)
        for l in range(L):
            pre = f"model.layers.{l}."
            xn = rms(x, from_bf16(t[pre + "input_layernorm.weight"]))
            q = proj(xn, pre + "self_attn.q_proj.weight").reshape(nq, D)
            k = proj(xn, pre + "self_attn.k_proj.weight").reshape(nk, D)
            v = proj(xn, pre + "self_attn.v_proj.weight").reshape(nk, D)
            ang = p * inv
            c, s = np.cos(ang), np.sin(ang)

            def rope(hd, w):
                hd = hd / np.sqrt(np.mean(hd * hd) + 1e-6) * w
                a, b = hd[:D // 2], hd[D // 2:]
                return np.concatenate([a * c - b * s, b * c + a * s])
            qn = from_bf16(t[pre + "self_attn.q_norm.weight"])
            kn = from_bf16(t[pre + "self_attn.k_norm.weight"])
            q = np.stack([rope(q[h], qn) for h in range(nq)])
            k = np.stack([rope(k[h], kn) for h in range(nk)])
            ks[l][ti], vs[l][ti] = k, v
            K = np.stack(ks[l][:ti + 1])
            Vv = np.stack(vs[l][:ti + 1])
            att = np.zeros((nq, D))
            for h in range(nq):
                sc = K[:, h // (nq // nk), :] @ q[h] / np.sqrt(D)
                pr = np.exp(sc - sc.max())
                pr /= pr.sum()
                att[h] = pr @ Vv[:, h // (nq // nk), :]
            x = x + proj(att.ravel(), pre + "self_attn.o_proj.weight")
            xn = rms(x, from_bf16(t[pre + "post_attention_layernorm.weight"]))
            g = proj(xn, pre + "mlp.gate_proj.weight")
            u = proj(xn, pre + "mlp.up_proj.weight")
            x = x + proj(g / (1 + np.exp(-g)) * u, pre + "mlp.down_proj.weight")
        x = rms(x, from_bf16(t["model.norm.weight"]))
        lm = t.get("lm_head.weight", t["model.embed_tokens.weight"])
        out = proj(x, orc.bf16_to_f16(lm).view(np.float16).astype(np.float64).reshape(V, H))
    return out


@pytest.mark.parametrize("tied", [True, False])
def test_qwen3_step_matches_float64_restatement(orc, rng, tied):
    t, d = tiny_model(rng, tied=tied)
    cfg = orc.Qwen3Config(d["H"], d["L"], d["nq"], d["nk"], d["D"], d["I"], d["V"], 1e6, 1e-6)
    B, steps = 2, 5
    m = orc.Qwen3(cfg, t, B, kv_capacity=64)
    toks = rng.integers(0, d["V"], (steps, B))
    pos0 = np.array([0, 20000])                      # the second sequence uses the RoPE fallback
    for s in range(steps):
        logits = m.forward(toks[s], pos0 + s)
    for b in range(B):
        ref = reference_step(orc, t, d, list(toks[:, b]), list(pos0[b] + np.arange(steps)))
        # fp16 rounding points: a value within an fp32 rounding of an fp16
        # tie can round differently; allow a few fp16 ulps of the logit scale
        err = np.max(np.abs(logits[b] - ref)) / np.max(np.abs(ref))
        assert err < 4e-3, err
