"""Comparison helpers with the tolerances the parity tests state."""
import numpy as np

# fp32 outputs of norm, RoPE and softmax: max relative error <= 1e-5
REL_TOL = 1e-5


def max_rel_err(got, ref, denom=None):
    got = np.asarray(got, np.float64)
    ref = np.asarray(ref, np.float64)
    d = np.abs(ref) if denom is None else np.asarray(denom, np.float64)
    d = np.maximum(d, np.finfo(np.float32).tiny)
    return float(np.max(np.abs(got - ref) / d)) if got.size else 0.0


def bits(a):
    a = np.ascontiguousarray(a)
    return a.view(np.uint32 if a.dtype.itemsize == 4 else np.uint16)


def assert_bitexact(got, ref, what=""):
    g, r = bits(got), bits(ref)
    bad = np.flatnonzero(g.ravel() != r.ravel())
    assert bad.size == 0, f"{what}: {bad.size} mismatches, first at {bad[:5]}: {g.ravel()[bad[:5]]} vs {r.ravel()[bad[:5]]}"


def attention_fp64(q, kc, vc, nq, nk, D, start, length, qs=None):
    """float64 GQA attention over ring positions (start + t) mod capacity.
    q flat (head h at h*qs); caches [capacity, nk*D].  Returns (out, bound):
    out [nq, D] and bound = sum_t p_t |v_t|, the scale of the terms summed,
    which the attention tolerances are relative to."""
    qs = D if qs is None else qs
    cap = kc.shape[0]
    if length <= 0:
        return np.zeros((nq, D)), np.zeros((nq, D))
    slots = (start + np.arange(length)) % cap
    K = kc.reshape(cap, nk, D)[slots].astype(np.float64)
    V = vc.reshape(cap, nk, D)[slots].astype(np.float64)
    out = np.zeros((nq, D))
    bound = np.zeros((nq, D))
    for h in range(nq):
        kv = h // (nq // nk)
        qh = q[h * qs:h * qs + D].astype(np.float64)
        s = (K[:, kv, :] @ qh) / np.sqrt(D)
        p = np.exp(s - s.max())
        p /= p.sum()
        out[h] = p @ V[:, kv, :]
        bound[h] = p @ np.abs(V[:, kv, :])
    return out, bound


# ---------------------------------------------------------------- tiny Qwen3 checkpoints

def bf16(a):
    """bf16 bits of the truncation of a float32 array (the model-building convention)"""
    return (np.ascontiguousarray(a, np.float32).view(np.uint32) >> 16).astype(np.uint16)


def from_bf16(b):
    return (b.astype(np.uint32) << 16).view(np.float32)


def tiny_qwen3(rng, H=256, L=2, nq=4, nk=2, D=128, I=384, V=300, tied=True):
    t = {"model.embed_tokens.weight": bf16(0.5 * rng.standard_normal((V, H))),
         "model.norm.weight": bf16(1 + 0.1 * rng.standard_normal(H))}
    for l in range(L):
        p = f"model.layers.{l}."
        t[p + "self_attn.q_proj.weight"] = bf16(0.06 * rng.standard_normal((nq * D, H)))
        t[p + "self_attn.k_proj.weight"] = bf16(0.06 * rng.standard_normal((nk * D, H)))
        t[p + "self_attn.v_proj.weight"] = bf16(0.06 * rng.standard_normal((nk * D, H)))
        t[p + "self_attn.o_proj.weight"] = bf16(0.06 * rng.standard_normal((H, nq * D)))
        t[p + "self_attn.q_norm.weight"] = bf16(1 + 0.1 * rng.standard_normal(D))
        t[p + "self_attn.k_norm.weight"] = bf16(1 + 0.1 * rng.standard_normal(D))
        t[p + "mlp.gate_proj.weight"] = bf16(0.06 * rng.standard_normal((I, H)))
        t[p + "mlp.up_proj.weight"] = bf16(0.06 * rng.standard_normal((I, H)))
        t[p + "mlp.down_proj.weight"] = bf16(0.06 * rng.standard_normal((H, I)))
        t[p + "input_layernorm.weight"] = bf16(1 + 0.1 * rng.standard_normal(H))
        t[p + "post_attention_layernorm.weight"] = bf16(1 + 0.1 * rng.standard_normal(H))
    if not tied:
        t["lm_head.weight"] = bf16(0.06 * rng.standard_normal((V, H)))
    return t, dict(H=H, L=L, nq=nq, nk=nk, D=D, I=I, V=V)



def save_qwen3(path, tensors):
    """Write bf16 bit arrays as a safetensors checkpoint."""
    import torch
    from safetensors.torch import save_file

    save_file({k: torch.from_numpy(np.ascontiguousarray(v).view(np.int16)).view(torch.bfloat16)
               for k, v in tensors.items()}, str(path))


# ---------------------------------------------------------------- GPU plumbing

def dev(a):
    """numpy -> torch tensor on cuda:0 (uint16 arrays travel as int16)."""
    import torch

    a = np.ascontiguousarray(a)
    if a.dtype == np.uint16:
        a = a.view(np.int16)
    return torch.from_numpy(a).cuda()


def host(t):
    import torch

    torch.cuda.synchronize()
    a = t.detach().cpu()
    if a.dtype in (torch.float16, torch.bfloat16):
        a = a.view(torch.int16)
    a = a.numpy()
    return a.view(np.uint16) if a.dtype == np.int16 else a


def f16_normal(rng, shape, std):
    """fp16 bits of the RNE fp16 of an fp32 N(0, std) draw."""
    return (rng.standard_normal(shape, dtype=np.float32) * np.float32(std)).astype(np.float16).view(np.uint16)


def gamma_f16(rng, n):
    """norm gammas ~ 1 + N(0, 0.02) stored as fp16 bits"""
    return (1.0 + rng.normal(0, 0.02, n)).astype(np.float32).astype(np.float16).view(np.uint16)


def rope_den(n, c, s, half):
    """|a c| + |b s| for the two halves of each head: the RoPE error scale.
    n: [..., 2*half] normalised (unrotated) heads; c, s: [..., half]."""
    a, b = n[..., :half].astype(np.float64), n[..., half:].astype(np.float64)
    c, s = np.abs(c.astype(np.float64)), np.abs(s.astype(np.float64))
    return np.concatenate([np.abs(a) * c + np.abs(b) * s, np.abs(b) * c + np.abs(a) * s], axis=-1)
