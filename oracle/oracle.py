"""numpy binding of the CPU oracle (liboracle.so).

TEST INFRASTRUCTURE ONLY: imported by tests/, __graft_entry__.smoke() and
the cpu_baseline leg of bench.py as the checker.  The product never uses it.
"""
from __future__ import annotations

import ctypes
import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
# ANELM_ORACLE_LIB names another build of the same library (the sanitizer build)
LIB_PATH = os.environ.get("ANELM_ORACLE_LIB") or os.path.join(HERE, "liboracle.so")

_P, _L, _I, _F, _S = ctypes.c_void_p, ctypes.c_long, ctypes.c_int, ctypes.c_float, ctypes.c_size_t
_U16 = ctypes.c_uint16

_SIGS = {
    "orc_bf16_to_f32": (_F, [_U16]),
    "orc_f32_to_bf16": (_U16, [_F]),
    "orc_f16_to_f32": (_F, [_U16]),
    "orc_f32_to_f16": (_U16, [_F]),
    "orc_bf16_to_f16": (_U16, [_U16]),
    "orc_bf16_to_f16_vec": (None, [_P, _P, _S, _I]),
    "orc_bf16_to_f32_vec": (None, [_P, _P, _S]),
    "orc_f16_to_f32_vec": (None, [_P, _P, _S]),
    "orc_norm_weight_vec": (None, [_P, _P, _S, _L]),
    "orc_rmsnorm": (None, [_P, _P, _P, _I, _F]),
    "orc_rmsnorm_rows": (None, [_P, _P, _P, _L, _I, _L, _L, _F, _I]),
    "orc_silu_vec": (None, [_P, _S]),
    "orc_mul_sigmoid": (None, [_P, _P, _S]),
    "orc_silu_mul": (None, [_P, _P, _P, _S, _I]),
    "orc_rope_inv_freq": (None, [_P, _I, _F]),
    "orc_rope_table": (None, [_P, _P, _I, _I, _F]),
    "orc_rope_qwen3": (None, [_P, _P, _I, _I, _I, _I, _F, _P, _P]),
    "orc_rope_cached": (None, [_P, _P, _I, _I, _I, _I, _I, _I, _I, _F, _P, _P]),
    "orc_qknorm_rope": (None, [_P, _P, _L, _L, _P, _P, _P, _P, _P, _I, _F, _L, _I, _I, _I, _F, _I]),
    "orc_residual_add": (None, [_P, _P, _S, _I]),
    "orc_embed_gather": (_I, [_P, _P, _I, _P, _L, _L, _L]),
    "orc_sampler_expf": (_F, [_F]),
    "orc_softmax": (None, [_P, _I]),
    "orc_softmax_shift": (_I, [_L]),
    "orc_sample_token": (_I, [_P, _I, _F, _F, _I, _F, _P, _I, _F, _P]),
    "orc_cdf_walk": (_I, [_P, _I, _F]),
    "orc_layer_chain": (None, [_L, _I, _I, _I, _I, _I, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P,
                               _P, _P, _I, _F, _F, _I]),
    "orc_max_threads": (_I, []),
    "orc_kv_ring_append": (_I, [_P, _P, _P, _P, _I, _P, _P, _I]),
    "orc_rmsnorm_gated": (None, [_P, _P, _P, _P, _I]),
    "orc_l2_normalize": (None, [_P, _I]),
    "orc_conv1d_update": (None, [_P, _P, _P, _P, _P, _I, _I]),
    "orc_ssm_step": (None, [_P, _P, _P, _P, _P, _F, _F, _I, _I]),
    "orc_matvec": (None, [_P, _P, _P, _I, _I]),
    "orc_f32_to_f16_rne": (_U16, [_F]),
    "orc_linear_f16": (None, [_P, _P, _P, _L, _I, _I]),
    "orc_qwen3_create": (_P, [_P, _I, _I, _P, _P, _P, _P]),
    "orc_qwen3_forward": (None, [_P, _P, _P, _P]),
    "orc_qwen3_free": (None, [_P]),
    "orc_gqa_attention": (None, [_P, _P, _P, _P, _I, _I, _I, _I, _I, _I, _I]),
}

_lib = None


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(f"{LIB_PATH} not built (make -C oracle)")
        l = ctypes.CDLL(LIB_PATH)
        for name, (res, args) in _SIGS.items():
            fn = getattr(l, name)
            fn.restype = res
            fn.argtypes = args
        _lib = l
    return _lib


def _p(a):
    return None if a is None else ctypes.c_void_p(a.ctypes.data)


def _c(a, dtype):
    a = np.ascontiguousarray(a, dtype=dtype)
    return a


# ---------------------------------------------------------------- converts

def bf16_to_f16(bits: np.ndarray, nthreads: int = 0) -> np.ndarray:
    src = _c(bits, np.uint16)
    out = np.empty_like(src)
    lib().orc_bf16_to_f16_vec(_p(out), _p(src), src.size, nthreads)
    return out


def f16_to_f32(bits: np.ndarray) -> np.ndarray:
    src = _c(bits, np.uint16)
    out = np.empty(src.shape, np.float32)
    lib().orc_f16_to_f32_vec(_p(out), _p(src), src.size)
    return out


def bf16_to_f32(bits: np.ndarray) -> np.ndarray:
    src = _c(bits, np.uint16)
    out = np.empty(src.shape, np.float32)
    lib().orc_bf16_to_f32_vec(_p(out), _p(src), src.size)
    return out


def norm_weight(bits: np.ndarray, expected_numel: int | None = None) -> np.ndarray:
    """Qwen3.5 (1+w) norm weight (core/safetensors.cpp:299-306): bf16 widened
    to fp32 plus 1.0f over the first expected_numel entries (default: all)."""
    src = _c(bits, np.uint16)
    out = np.empty(src.shape, np.float32)
    lib().orc_norm_weight_vec(_p(out), _p(src), src.size, src.size if expected_numel is None else expected_numel)
    return out


def f32_to_f16_scalar(x: float) -> int:
    return lib().orc_f32_to_f16(x)


def f32_to_bf16(x: np.ndarray) -> np.ndarray:
    """Truncating fp32 -> bf16 bits (include/ane_lm/common.h:28-32)."""
    return (_c(x, np.float32).view(np.uint32) >> 16).astype(np.uint16)


# ---------------------------------------------------------------- norms

def rmsnorm_rows(x: np.ndarray, w: np.ndarray, eps: float = 1e-6, nthreads: int = 0) -> np.ndarray:
    x = _c(x, np.float32)
    w = _c(w, np.float32)
    rows, dim = x.shape
    out = np.empty_like(x)
    lib().orc_rmsnorm_rows(_p(out), _p(x), _p(w), rows, dim, dim, dim, eps, nthreads)
    return out


def rmsnorm(x: np.ndarray, w: np.ndarray, eps: float = 1e-6) -> np.ndarray:
    x = _c(x, np.float32)
    out = np.empty_like(x)
    lib().orc_rmsnorm(_p(out), _p(x), _p(_c(w, np.float32)), x.size, eps)
    return out


def silu(x: np.ndarray) -> np.ndarray:
    y = _c(x, np.float32).copy()
    lib().orc_silu_vec(_p(y), y.size)
    return y


def mul_sigmoid(y: np.ndarray, z: np.ndarray) -> np.ndarray:
    y = _c(y, np.float32).copy()
    z = _c(z, np.float32)
    lib().orc_mul_sigmoid(_p(y), _p(z), y.size)
    return y


def silu_mul(g: np.ndarray, u: np.ndarray, nthreads: int = 0) -> np.ndarray:
    g = _c(g, np.float32)
    u = _c(u, np.float32)
    h = np.empty_like(g)
    lib().orc_silu_mul(_p(h), _p(g), _p(u), g.size, nthreads)
    return h


def residual_add(x: np.ndarray, y: np.ndarray, nthreads: int = 0) -> np.ndarray:
    x = _c(x, np.float32).copy()
    lib().orc_residual_add(_p(x), _p(_c(y, np.float32)), x.size, nthreads)
    return x


# ---------------------------------------------------------------- RoPE

def rope_inv_freq(rot_dim: int, theta: float) -> np.ndarray:
    out = np.empty(rot_dim // 2, np.float32)
    lib().orc_rope_inv_freq(_p(out), rot_dim, theta)
    return out


def rope_table(n_pos: int, rot_dim: int, theta: float):
    c = np.empty((n_pos, rot_dim // 2), np.float32)
    s = np.empty_like(c)
    lib().orc_rope_table(_p(c), _p(s), n_pos, rot_dim, theta)
    return c, s


def qknorm_rope(q, k, wq, wk, pos, cos_tab, sin_tab, theta, nq, nk, head_dim, eps=1e-6, nthreads=0):
    """q: [T, q_ld], k: [T, k_ld] (copied); returns (q', k')."""
    q = _c(q, np.float32).copy()
    k = _c(k, np.float32).copy()
    pos = _c(pos, np.int32)
    T = pos.shape[0]
    tab_len = 0 if cos_tab is None else cos_tab.shape[0]
    lib().orc_qknorm_rope(_p(q), _p(k), q.shape[1], k.shape[1], _p(None if wq is None else _c(wq, np.float32)),
                          _p(None if wk is None else _c(wk, np.float32)), _p(pos),
                          _p(None if cos_tab is None else _c(cos_tab, np.float32)),
                          _p(None if sin_tab is None else _c(sin_tab, np.float32)), tab_len, theta, T, nq, nk,
                          head_dim, eps, nthreads)
    return q, k


def rope_cached(q, k, n_q_heads, n_kv_heads, head_dim, q_head_stride, k_head_stride, rot_dim, pos, theta,
                cos_row=None, sin_row=None):
    q = _c(q, np.float32).copy()
    k = _c(k, np.float32).copy()
    lib().orc_rope_cached(_p(q), _p(k), n_q_heads, n_kv_heads, head_dim, q_head_stride, k_head_stride, rot_dim,
                          pos, theta, _p(None if cos_row is None else _c(cos_row, np.float32)),
                          _p(None if sin_row is None else _c(sin_row, np.float32)))
    return q, k


# ---------------------------------------------------------------- gather

def embed_gather(table: np.ndarray, ids: np.ndarray, dtype_code: int):
    """dtype_code 0 fp32 table, 1 fp16 bits, 2 bf16 bits."""
    table = np.ascontiguousarray(table)
    ids = _c(ids, np.int32)
    vocab, hidden = table.shape
    out = np.empty((ids.shape[0], hidden), np.float32)
    rc = lib().orc_embed_gather(_p(out), _p(table), dtype_code, _p(ids), ids.shape[0], hidden, vocab)
    if rc != 0:
        raise IndexError("embedding id out of range")
    return out


# ---------------------------------------------------------------- sampling

def sampler_expf(x: float) -> float:
    return lib().orc_sampler_expf(x)


def softmax(x: np.ndarray) -> np.ndarray:
    y = _c(x, np.float32).copy()
    lib().orc_softmax(_p(y), y.size)
    return y


def softmax_shift(n: int) -> int:
    return lib().orc_softmax_shift(n)


def sample_token(logits: np.ndarray, temperature=0.6, repetition_penalty=1.2, repetition_context_size=256,
                 frequency_penalty=0.1, recent=None, r=0.0, want_probs=False):
    logits = _c(logits, np.float32)
    V = logits.size
    rec = _c(recent if recent is not None else np.zeros(0, np.int32), np.int32)
    probs = np.empty(V, np.float32) if want_probs else None
    tok = lib().orc_sample_token(_p(logits), V, temperature, repetition_penalty, repetition_context_size,
                                 frequency_penalty, _p(rec) if rec.size else None, rec.size, r, _p(probs))
    return (tok, probs) if want_probs else tok


def cdf_walk(p: np.ndarray, r: float) -> int:
    p = _c(p, np.float32)
    return lib().orc_cdf_walk(_p(p), p.size, r)


def layer_chain(T, H, nq, nk, D, I, x, xn, attn_out, mlp_out, q, k, g, u, h, w_in, w_post, wq, wk, pos, cos_tab,
                sin_tab, theta, eps, nthreads=0):
    """In place on x, xn, q, k, h (contiguous float32 numpy arrays)."""
    lib().orc_layer_chain(T, H, nq, nk, D, I, _p(x), _p(xn), _p(attn_out), _p(mlp_out), _p(q), _p(k), _p(g), _p(u),
                          _p(h), _p(w_in), _p(w_post), _p(wq), _p(wk), _p(pos), _p(cos_tab), _p(sin_tab),
                          cos_tab.shape[0], theta, eps, nthreads)


def kv_ring_append(k_cache, v_cache, k, v, state):
    """Append rows k, v ([n_kv_heads*head_dim] each) to the ring caches
    [capacity, kv_stride] in place; state = [start, len] (np.int32, updated).
    Returns the slot written."""
    cap, stride = k_cache.shape
    assert state.dtype == np.int32 and state.size == 2 and state.flags.c_contiguous
    assert k_cache.flags.c_contiguous and v_cache.flags.c_contiguous and k_cache.dtype == np.float32
    return lib().orc_kv_ring_append(_p(k_cache), _p(v_cache), _p(_c(k, np.float32)), _p(_c(v, np.float32)), stride,
                                    ctypes.c_void_p(state.ctypes.data), ctypes.c_void_p(state.ctypes.data + 4), cap)


def gqa_attention(q, k_cache, v_cache, n_heads, n_kv_heads, head_dim, cache_start, cache_len, q_head_stride=None):
    """q: flat [>= (n_heads-1)*q_head_stride + head_dim]; caches [capacity,
    n_kv_heads*head_dim] (or any shape of that size).  Returns [n_heads, head_dim]."""
    q = _c(q, np.float32).ravel()
    kc, vc = _c(k_cache, np.float32), _c(v_cache, np.float32)
    cap = kc.size // (n_kv_heads * head_dim)
    qs = head_dim if q_head_stride is None else q_head_stride
    out = np.empty((n_heads, head_dim), np.float32)
    lib().orc_gqa_attention(_p(out), _p(q), _p(kc), _p(vc), n_heads, n_kv_heads, head_dim, qs, cache_start,
                            cache_len, cap)
    return out


def rmsnorm_gated(x, z, w):
    x, z, w = _c(x, np.float32), _c(z, np.float32), _c(w, np.float32)
    out = np.empty_like(x)
    lib().orc_rmsnorm_gated(_p(out), _p(x), _p(z), _p(w), x.size)
    return out


def l2_normalize(x):
    y = _c(x, np.float32).copy()
    lib().orc_l2_normalize(_p(y), y.size)
    return y


def conv1d_update(conv_state, state_pos, x, w):
    """conv_state [channels, K-1] float32 (updated in place); state_pos an
    np.int32 array of one element (updated); w [channels, K]. Returns y."""
    ch, K = w.shape
    assert conv_state.flags.c_contiguous and conv_state.dtype == np.float32 and conv_state.shape == (ch, K - 1)
    assert state_pos.dtype == np.int32 and state_pos.size == 1
    y = np.empty(ch, np.float32)
    lib().orc_conv1d_update(_p(y), _p(conv_state), ctypes.c_void_p(state_pos.ctypes.data), _p(_c(x, np.float32)),
                            _p(_c(w, np.float32)), ch, K)
    return y


def ssm_step(state, q, k, v, decay, beta):
    """state [key_dim, value_dim] float32, updated in place. Returns y."""
    kd, vd = state.shape
    assert state.flags.c_contiguous and state.dtype == np.float32
    y = np.empty(vd, np.float32)
    lib().orc_ssm_step(_p(y), _p(state), _p(_c(q, np.float32)), _p(_c(k, np.float32)), _p(_c(v, np.float32)),
                       decay, beta, kd, vd)
    return y


def matvec(W, x):
    W, x = _c(W, np.float32), _c(x, np.float32)
    y = np.empty(W.shape[0], np.float32)
    lib().orc_matvec(_p(y), _p(W), _p(x), W.shape[0], W.shape[1])
    return y


def max_threads() -> int:
    return lib().orc_max_threads()


# ------------------------------------------------------------ safetensors, ANE blobs

ST_DTYPES = {"BF16": (np.uint16, 2), "F16": (np.uint16, 2), "F32": (np.float32, 4), "F64": (np.float64, 8),
             "I32": (np.int32, 4), "I64": (np.int64, 8), "U8": (np.uint8, 1)}


def read_safetensors(path):
    """{name: (dtype string, shape, raw data as a numpy array)} in header
    order: an 8-byte little-endian header length, a JSON header, then the
    data block (the format core/safetensors.cpp:193-244 reads).  BF16/F16
    data are returned as uint16 bit patterns; "__metadata__" is skipped."""
    import json

    with open(path, "rb") as f:
        blob = f.read()
    hlen = int.from_bytes(blob[:8], "little")
    header = json.loads(blob[8:8 + hlen])
    base = 8 + hlen
    out = {}
    for name, info in header.items():
        if name == "__metadata__":
            continue
        a, b = info["data_offsets"]
        dt, size = ST_DTYPES.get(info["dtype"], (np.uint8, 1))
        out[name] = (info["dtype"], tuple(info["shape"]), np.frombuffer(blob[base + a:base + b], dtype=dt))
    return out


def ane_blob(bf16_bits):
    """The ANE weight blob of a BF16 tensor, core/safetensors.cpp:316-343
    (same bytes as core/ane_runtime.cpp:195-209): a 64-byte global header
    with byte 0 = 1 and byte 4 = 2, a 64-byte chunk header with magic
    EF BE AD DE, version 1 at +4, the fp16 data size (u32 LE) at +8 and the
    data offset 128 (u32 LE) at +16, zeros elsewhere; then the truncating
    fp16 convert of the data (common.h:81-83)."""
    bits = np.ascontiguousarray(bf16_bits, dtype=np.uint16).ravel()
    hdr = bytearray(128)
    hdr[0] = 0x01
    hdr[4] = 0x02
    hdr[64:68] = bytes([0xEF, 0xBE, 0xAD, 0xDE])
    hdr[68] = 0x01
    hdr[72:76] = (bits.size * 2 & 0xFFFFFFFF).to_bytes(4, "little")
    hdr[80:84] = (128).to_bytes(4, "little")
    return bytes(hdr) + bf16_to_f16(bits).tobytes()


def blob_relpath(name):
    """core/safetensors.cpp:355-361: dots become directory separators, plus ".bin"."""
    return name.replace(".", "/") + ".bin"


def write_ane_blobs(st_path, out_dir):
    """core/safetensors.cpp:345-383: one blob per BF16 tensor.  Returns the count."""
    n = 0
    for name, (dt, shape, data) in read_safetensors(st_path).items():
        if dt != "BF16":
            continue
        p = os.path.join(out_dir, blob_relpath(name))
        os.makedirs(os.path.dirname(p), exist_ok=True)
        with open(p, "wb") as f:
            f.write(ane_blob(data))
        n += 1
    return n


# ------------------------------------------------------------ ANE contractions, Qwen3 step

class Qwen3Config(ctypes.Structure):
    _fields_ = [("hidden", ctypes.c_int), ("layers", ctypes.c_int), ("n_q_heads", ctypes.c_int),
                ("n_kv_heads", ctypes.c_int), ("head_dim", ctypes.c_int), ("intermediate", ctypes.c_int),
                ("vocab", ctypes.c_int), ("rope_theta", ctypes.c_float), ("rms_eps", ctypes.c_float)]


def f32_to_f16_rne(x: np.ndarray) -> np.ndarray:
    x = _c(x, np.float32).ravel()
    f = lib().orc_f32_to_f16_rne
    return np.array([f(float(v)) for v in x], np.uint16)


def linear_f16(x16, w16):
    """y16 [batch, out] = fp16_rne(x16 @ w16.T) with exact accumulation (fp16 bit arrays)."""
    x16 = _c(x16, np.uint16)
    w16 = _c(w16, np.uint16)
    batch = x16.shape[0] if x16.ndim == 2 else 1
    out_dim, in_dim = w16.shape
    y = np.empty((batch, out_dim), np.uint16)
    lib().orc_linear_f16(_p(y), _p(x16), _p(w16), batch, out_dim, in_dim)
    return y


QWEN3_LAYER_TENSORS = ["self_attn.q_proj.weight", "self_attn.k_proj.weight", "self_attn.v_proj.weight",
                       "self_attn.o_proj.weight", "self_attn.q_norm.weight", "self_attn.k_norm.weight",
                       "mlp.gate_proj.weight", "mlp.up_proj.weight", "mlp.down_proj.weight",
                       "input_layernorm.weight", "post_attention_layernorm.weight"]


class Qwen3:
    """The oracle's Qwen3 decode step over `batch` sequences from a dict of
    bf16 bit arrays keyed by the checkpoint's tensor names."""

    def __init__(self, cfg: Qwen3Config, tensors: dict, batch: int, kv_capacity: int):
        self._keep = {k: _c(v, np.uint16) for k, v in tensors.items()}
        ptrs = []
        for L in range(cfg.layers):
            for n in QWEN3_LAYER_TENSORS:
                ptrs.append(self._keep[f"model.layers.{L}.{n}"].ctypes.data)
        arr = (ctypes.c_void_p * len(ptrs))(*ptrs)
        self._arr = arr
        self.cfg, self.batch = cfg, batch
        lm = self._keep.get("lm_head.weight")
        self._h = lib().orc_qwen3_create(ctypes.byref(cfg), batch, kv_capacity,
                                         _p(self._keep["model.embed_tokens.weight"]), arr,
                                         _p(self._keep["model.norm.weight"]), _p(lm) if lm is not None else None)

    def forward(self, ids, pos):
        ids = _c(ids, np.int32)
        pos = _c(pos, np.int32)
        out = np.empty((self.batch, self.cfg.vocab), np.float32)
        lib().orc_qwen3_forward(self._h, _p(ids), _p(pos), _p(out))
        return out

    def __del__(self):
        if getattr(self, "_h", None):
            lib().orc_qwen3_free(self._h)
            self._h = None
