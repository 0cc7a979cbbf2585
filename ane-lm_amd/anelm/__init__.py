"""ctypes binding of libanelm_hip.so for Python callers (tests, bench).

PyTorch is used only for device memory and streams: every function takes
torch tensors that already live on the GPU, passes their raw device
pointers and the current HIP stream to the C ABI (include/anelm_hip.h),
and raises AnelmError with the library's message on a non-zero status.
There is no fallback: if the library is missing or fails, the call raises.
"""
from __future__ import annotations

import ctypes
import os

_PKG = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
# ANELM_LIB names another build of the same library (the host-sanitizer build)
LIB_PATH = os.environ.get("ANELM_LIB") or os.path.join(_PKG, "lib", "libanelm_hip.so")

F32, F16, BF16 = 0, 1, 2
OK, ERR_INVALID, ERR_RANGE, ERR_HIP, ERR_WORKSPACE = 0, -1, -2, -3, -4


class AnelmError(RuntimeError):
    def __init__(self, code: int, msg: str):
        super().__init__(f"anelm error {code}: {msg}")
        self.code = code


class SamplingParams(ctypes.Structure):
    """anelm_sampling_params; defaults of core/sampling.h:7-12."""

    _fields_ = [
        ("temperature", ctypes.c_float),
        ("repetition_penalty", ctypes.c_float),
        ("repetition_context_size", ctypes.c_int),
        ("frequency_penalty", ctypes.c_float),
    ]

    def __init__(self, temperature=0.6, repetition_penalty=1.2, repetition_context_size=256,
                 frequency_penalty=0.1):
        super().__init__(temperature, repetition_penalty, repetition_context_size, frequency_penalty)


_lib = None
_P = ctypes.c_void_p
_L = ctypes.c_long
_I = ctypes.c_int
_F = ctypes.c_float
_S = ctypes.c_size_t

_SIGS = {
    "anelm_last_error": (ctypes.c_char_p, []),
    "anelm_version": (_I, []),
    "anelm_rmsnorm": (_I, [_P, _P, _P, _I, _L, _I, _L, _L, _F, _P]),
    "anelm_rmsnorm_geometry": (_I, [_L, _I, ctypes.POINTER(_I), ctypes.POINTER(_I)]),
    "anelm_rmsnorm_f16": (_I, [_P, _P, _P, _I, _L, _I, _L, _L, _F, _P]),
    "anelm_rmsnorm_f16_tiled": (_I, [_P, _P, _P, _I, _L, _I, _L, _F, _P]),
    "anelm_add_rmsnorm": (_I, [_P, _P, _P, _P, _I, _L, _I, _L, _L, _L, _F, _P]),
    "anelm_qknorm_rope": (_I, [_P, _P, _L, _L, _P, _P, _I, _P, _P, _P, _I, _F, _L, _I, _I, _I, _F, _P]),
    "anelm_qknorm_rope_append": (_I, [_P, _P, _P, _L, _L, _L, _P, _P, _I, _P, _P, _P, _I, _F, _L, _I, _I, _F, _P, _P,
                                      _P, _P, _I, _L, _P]),
    "anelm_rope_cached": (_I, [_P, _P, _I, _I, _I, _I, _I, _I, _I, _F, _P, _P, _P]),
    "anelm_rope_table": (_I, [_P, _P, _I, _I, _F, _P]),
    "anelm_residual_add": (_I, [_P, _P, _S, _P]),
    "anelm_silu_mul": (_I, [_P, _P, _P, _L, _L, _L, _L, _L, _P]),
    "anelm_silu": (_I, [_P, _S, _P]),
    "anelm_mul_sigmoid": (_I, [_P, _P, _S, _P]),
    "anelm_embed_gather": (_I, [_P, _P, _I, _P, _L, _L, _L, _P, _P]),
    "anelm_bf16_to_f16": (_I, [_P, _P, _S, _P]),
    "anelm_bf16_to_f32": (_I, [_P, _P, _S, _P]),
    "anelm_bf16_to_f32_plus1": (_I, [_P, _P, _S, _P]),
    "anelm_bf16_to_f16_multi": (_I, [_P, _P, _P, _I, _P]),
    "anelm_f16_to_f32": (_I, [_P, _P, _S, _P]),
    "anelm_f32_to_f16": (_I, [_P, _P, _S, _P]),
    "anelm_softmax_workspace_size": (_S, [_L, _L]),
    "anelm_softmax": (_I, [_P, _L, _L, _L, _P, _S, _P]),
    "anelm_sample_workspace_size": (_S, [_L, _L]),
    "anelm_sample": (_I, [_P, _P, _L, _P, _L, _L, _L, _P, _L, _P, ctypes.POINTER(SamplingParams), _P, _P, _S, _P]),
    "anelm_layer_ops": (_I, [_P] * 14 + [_I, _P, _P, _P, _I, _F, _L, _I, _I, _I, _L, _F, _P]),
    "anelm_sample_noalloc": (_I, [_P, _P, _L, _P, _L, _L, _L, _P, _L, _P, ctypes.POINTER(SamplingParams), _P, _P]),
    "anelm_gqa_workspace_size": (_S, [_L, _I, _I, _I, _I]),
    "anelm_gqa_attention": (_I, [_P, _P, _P, _P, _P, _P, _L, _I, _I, _I, _L, _I, _L, _I, _L, _P, _S, _P]),
    "anelm_gqa_attention_f16": (_I, [_P, _P, _P, _P, _P, _P, _L, _I, _I, _I, _L, _I, _L, _I, _L, _P, _S, _P]),
    "anelm_gqa_attention_bounded": (_I, [_P, _P, _P, _P, _P, _P, _L, _I, _I, _I, _L, _I, _L, _I, _L, _I, _P, _S,
                                         _P]),
    "anelm_gqa_attention_ring": (_I, [_P, _P, _P, _P, _I, _I, _I, _I, _I, _I, _I, _P, _S, _P]),
    "anelm_kv_ring_append": (_I, [_P, _P, _P, _P, _P, _P, _L, _L, _L, _I, _I, _I, _L, _P]),
    "anelm_kv_ring_advance": (_I, [_P, _P, _L, _I, _L, _I, _P]),
    "anelm_gqa_attention_qk": (_I, [_P, _I, _P, _P, _P, _L, _L, _L, _P, _P, _I, _P, _P, _P, _I, _F, _F, _P, _P, _P, _P,
                                    _L, _I, _I, _L, _I, _L, _P, _S, _P]),
    "anelm_gqa_attention_qk_append": (_I, [_P, _I, _P, _P, _P, _L, _L, _L, _P, _P, _I, _P, _P, _P, _I, _F, _F, _P, _P,
                                           _P, _P, _L, _I, _I, _L, _I, _L, _P, _S, _P]),
    "anelm_rmsnorm_gated": (_I, [_P, _P, _P, _P, _I, _L, _I, _I, _L, _L, _L, _F, _P]),
    "anelm_l2_normalize": (_I, [_P, _L, _I, _I, _L, _F, _P]),
    "anelm_conv1d_update": (_I, [_P, _P, _P, _P, _P, _L, _I, _I, _L, _L, _L, _P]),
    "anelm_ssm_step": (_I, [_P, _P, _P, _P, _P, _P, _P, _L, _I, _I, _I, _I, _L, _L, _L, _L, _P]),
    "anelm_ssm_step_gated_norm": (_I, [_P, _P, _P, _P, _P, _P, _P, _P, _P, _I, _L, _I, _I, _I, _I, _L, _L, _L, _L,
                                       _L, _F, _P]),
    "anelm_conv1d_silu_l2norm": (_I, [_P, _P, _P, _P, _P, _L, _I, _I, _L, _L, _L, _F, _P]),
    "anelm_conv_ssm_step_gated_norm": (_I, [_P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _I, _L, _I, _L, _L, _L, _L, _L,
                                            _F, _F, _P]),
    "anelm_matvec": (_I, [_P, _P, _P, _L, _I, _P]),
    "anelm_st_open": (_P, [ctypes.c_char_p]),
    "anelm_st_close": (None, [_P]),
    "anelm_st_count": (_L, [_P]),
    "anelm_st_find": (_L, [_P, ctypes.c_char_p]),
    "anelm_st_info": (_I, [_P, _L, ctypes.POINTER(ctypes.c_char_p), ctypes.POINTER(_I), ctypes.POINTER(_I),
                           ctypes.POINTER(ctypes.c_int64), ctypes.POINTER(ctypes.c_uint64),
                           ctypes.POINTER(ctypes.c_uint64)]),
    "anelm_st_host_data": (_P, [_P, _L]),
    "anelm_st_load": (_I, [_P, _L, _P, _I, _P]),
    "anelm_st_load_norm": (_I, [_P, _L, _P, _L, _P]),
    "anelm_ane_blob_header": (None, [_P, ctypes.c_uint64]),
    "anelm_write_ane_blobs": (_L, [ctypes.c_char_p, ctypes.c_char_p, _P]),
    "anelm_linear_f16": (_I, [_P, _P, _P, _L, _I, _I, _L, _L, _P]),
    "anelm_proj_f16": (_I, [_P, _P, _P, _L, _I, _I, _L, _L, _P]),
    "anelm_proj_f16_x16": (_I, [_P, _P, _P, _L, _I, _I, _L, _L, _P]),
    "anelm_proj_f16_fused": (_I, [_P, _P, _P, _L, _I, _I, _L, _L, _P, _F, _I, _P]),
    "anelm_proj_f16_x16_fused": (_I, [_P, _P, _P, _L, _I, _I, _L, _L, _I, _P]),
    "anelm_proj_tiled_size": (_S, [_I, _I]),
    "anelm_proj_tile_f16": (_I, [_P, _P, _I, _I, _P]),
    "anelm_proj_f16_x16_tiled": (_I, [_P, _P, _P, _L, _I, _I, _L, _L, _I, _P]),
    "anelm_proj_f16_tt": (_I, [_P, _P, _P, _L, _I, _I, _L, _I, _P]),
    "anelm_qwen3_load": (_P, [ctypes.c_char_p, _P, _I, _I, _P]),
    "anelm_qwen3_free": (None, [_P]),
    "anelm_qwen3_reset": (_I, [_P, _P]),
    "anelm_qwen3_forward": (_I, [_P, _P, _P, _L, _P, _L, _P, _P]),
}

EXPORTED = tuple(_SIGS)


def lib():
    """Load libanelm_hip.so (after torch, so both share torch's HIP runtime)."""
    global _lib
    if _lib is not None:
        return _lib
    import torch  # noqa: F401  -- torch's libamdhip64.so.7 must be the one in the process

    if not os.path.exists(LIB_PATH):
        raise AnelmError(ERR_HIP, f"{LIB_PATH} is not built (python ane-lm_amd/build.py)")
    l = ctypes.CDLL(LIB_PATH)
    for name, (res, args) in _SIGS.items():
        fn = getattr(l, name)
        fn.restype = res
        fn.argtypes = args
    _lib = l
    return l


def last_error() -> str:
    return lib().anelm_last_error().decode()


def _check(rc: int) -> None:
    if rc != 0:
        raise AnelmError(rc, last_error())


def _ptr(t):
    return None if t is None else ctypes.c_void_p(t.data_ptr())


def _stream(stream):
    import torch

    if stream is None:
        stream = torch.cuda.current_stream()
    return ctypes.c_void_p(stream.cuda_stream)


def _dtype_code(t) -> int:
    import torch

    return {torch.float32: F32, torch.float16: F16, torch.bfloat16: BF16}[t.dtype]


def _need(cond: bool, msg: str) -> None:
    if not cond:
        raise AnelmError(ERR_INVALID, msg)


def _ld(x):
    """Row stride of a 2-D tensor; a single row's stride is arbitrary
    (numpy/torch may report 0 for it), so the row length stands in."""
    return x.stride(0) if x.shape[0] > 1 else x.shape[1]


def _rows(x):
    """(rows, dim, ld) of a 2-D tensor with unit inner stride."""
    _need(x.dim() == 2 and (x.stride(1) == 1 or x.shape[1] == 1), "expected a 2-D tensor with unit inner stride")
    return x.shape[0], x.shape[1], _ld(x)


# ---------------------------------------------------------------- ops

def rmsnorm(out, x, w, eps=1e-6, stream=None):
    rows, dim, ldx = _rows(x)
    _, _, ldo = _rows(out)
    _check(lib().anelm_rmsnorm(_ptr(out), _ptr(x), _ptr(w), _dtype_code(w), rows, dim, ldx, ldo, eps,
                               _stream(stream)))


def rmsnorm_geometry(rows, dim):
    """(float4 per lane, lanes per row) that rmsnorm and layer_ops launch
    with for rows of dim floats; (0, 256) for the any-shape kernel."""
    nv, thr = _I(), _I()
    _check(lib().anelm_rmsnorm_geometry(rows, dim, ctypes.byref(nv), ctypes.byref(thr)))
    return nv.value, thr.value


def rmsnorm_f16(out16, x, w, eps=1e-6, stream=None):
    """out16 (int16/float16 tensor, fp16 bits) = fp16 RNE of rmsnorm(x) * w."""
    rows, dim, ldx = _rows(x)
    _, _, ldo = _rows(out16)
    _check(lib().anelm_rmsnorm_f16(_ptr(out16), _ptr(x), _ptr(w), _dtype_code(w), rows, dim, ldx, ldo, eps,
                                   _stream(stream)))


def rmsnorm_f16_tiled(out_t, x, w, eps=1e-6, stream=None):
    """out_t (int16/float16, proj_tiled_size(rows, dim) bytes) = rmsnorm_f16 of x
    in the tiled layout of proj_tile_f16."""
    rows, dim, ldx = _rows(x)
    _need(_nbytes(out_t) >= lib().anelm_proj_tiled_size(rows, dim), "rmsnorm_f16_tiled: out_t too small")
    _check(lib().anelm_rmsnorm_f16_tiled(_ptr(out_t), _ptr(x), _ptr(w), _dtype_code(w), rows, dim, ldx, eps,
                                         _stream(stream)))


def add_rmsnorm(x, y, out, w, eps=1e-6, stream=None):
    rows, dim, ldx = _rows(x)
    _, _, ldy = _rows(y)
    _, _, ldo = _rows(out)
    _check(lib().anelm_add_rmsnorm(_ptr(x), _ptr(y), _ptr(out), _ptr(w), _dtype_code(w), rows, dim, ldx, ldy,
                                   ldo, eps, _stream(stream)))


def qknorm_rope(q, k, wq, wk, pos, cos_tab, sin_tab, theta=1e6, eps=1e-6, nq=None, nk=None, head_dim=128,
                stream=None):
    """q: [T, >= nq*head_dim] rows, k: [T, >= nk*head_dim] rows (views allowed)."""
    T = pos.shape[0]
    q_ld = _ld(q) if q is not None else 0
    k_ld = _ld(k) if k is not None else 0
    nq = (q.shape[1] // head_dim if q is not None else 0) if nq is None else nq
    nk = (k.shape[1] // head_dim if k is not None else 0) if nk is None else nk
    wdt = _dtype_code(wq if wq is not None else (wk if wk is not None else q))
    tab_len = cos_tab.shape[0] if cos_tab is not None else 0
    _check(lib().anelm_qknorm_rope(_ptr(q), _ptr(k), q_ld, k_ld, _ptr(wq), _ptr(wk), wdt, _ptr(pos), _ptr(cos_tab),
                                   _ptr(sin_tab), tab_len, theta, T, nq, nk, head_dim, eps, _stream(stream)))


def qknorm_rope_append(q, k, v, wq, wk, pos, cos_tab, sin_tab, k_cache, v_cache, ring_start, ring_len, theta=1e6,
                       eps=1e-6, nq=None, nk=None, stream=None):
    """Decode step: q/k norm + RoPE of token b (pos[b]) in place, then k and v
    appended to ring b; head_dim 128; caches [B, capacity, nk*128]."""
    B = pos.shape[0]
    nq = q.shape[1] // 128 if nq is None else nq
    nk = k.shape[1] // 128 if nk is None else nk
    _, cap, row = k_cache.shape
    _need(row == nk * 128 and k_cache.stride() == v_cache.stride(), "qknorm_rope_append: cache shapes")
    wdt = _dtype_code(wq if wq is not None else (wk if wk is not None else q))
    tab_len = cos_tab.shape[0] if cos_tab is not None else 0
    _check(lib().anelm_qknorm_rope_append(_ptr(q), _ptr(k), _ptr(v), _ld(q), _ld(k), _ld(v), _ptr(wq), _ptr(wk), wdt,
                                          _ptr(pos), _ptr(cos_tab), _ptr(sin_tab), tab_len, theta, B, nq, nk, eps,
                                          _ptr(k_cache), _ptr(v_cache), _ptr(ring_start), _ptr(ring_len), cap,
                                          k_cache.stride(0), _stream(stream)))


def rope_cached(q, k, n_q_heads, n_kv_heads, head_dim, q_head_stride, k_head_stride, rot_dim, pos, theta,
                cos_row=None, sin_row=None, stream=None):
    _check(lib().anelm_rope_cached(_ptr(q), _ptr(k), n_q_heads, n_kv_heads, head_dim, q_head_stride,
                                   k_head_stride, rot_dim, pos, theta, _ptr(cos_row), _ptr(sin_row),
                                   _stream(stream)))


def rope_table(cos_tab, sin_tab, theta=1e6, stream=None):
    n_pos, half = cos_tab.shape
    _check(lib().anelm_rope_table(_ptr(cos_tab), _ptr(sin_tab), n_pos, 2 * half, theta, _stream(stream)))


def residual_add(x, y, stream=None):
    _need(x.numel() == y.numel() and x.is_contiguous() and y.is_contiguous(), "residual_add: shapes")
    _check(lib().anelm_residual_add(_ptr(x), _ptr(y), x.numel(), _stream(stream)))


def silu_mul(h, g, u, stream=None):
    rows, inter, ldg = _rows(g)
    _, _, ldu = _rows(u)
    _, _, ldh = _rows(h)
    _check(lib().anelm_silu_mul(_ptr(h), _ptr(g), _ptr(u), rows, inter, ldh, ldg, ldu, _stream(stream)))


def silu(x, stream=None):
    _check(lib().anelm_silu(_ptr(x), x.numel(), _stream(stream)))


def mul_sigmoid(y, z, stream=None):
    _check(lib().anelm_mul_sigmoid(_ptr(y), _ptr(z), y.numel(), _stream(stream)))


def embed_gather(out, table, ids, bad_count=None, stream=None):
    vocab, hidden = table.shape
    _check(lib().anelm_embed_gather(_ptr(out), _ptr(table), _dtype_code(table), _ptr(ids), ids.shape[0], hidden, vocab,
                                    _ptr(bad_count), _stream(stream)))


def bf16_to_f16(dst, src, stream=None):
    """dst/src: uint16/int16 (or bf16/f16) tensors of the same element count."""
    _check(lib().anelm_bf16_to_f16(_ptr(dst), _ptr(src), src.numel(), _stream(stream)))


def bf16_to_f32(dst, src, stream=None):
    _check(lib().anelm_bf16_to_f32(_ptr(dst), _ptr(src), src.numel(), _stream(stream)))


def bf16_to_f16_multi(dsts, srcs, stream=None):
    """anelm_bf16_to_f16 over lists of tensors (uint16/int16 views), a few launches in all."""
    _need(len(dsts) == len(srcs), "bf16_to_f16_multi: list lengths")
    k = len(srcs)
    d = (ctypes.c_void_p * max(k, 1))(*[t.data_ptr() for t in dsts])
    sp = (ctypes.c_void_p * max(k, 1))(*[t.data_ptr() for t in srcs])
    n = (ctypes.c_size_t * max(k, 1))(*[t.numel() for t in srcs])
    _check(lib().anelm_bf16_to_f16_multi(d, sp, n, k, _stream(stream)))


def bf16_to_f32_plus1(dst, src, stream=None):
    """The Qwen3.5 (1+w) norm weight: dst = widen(src) + 1.0f."""
    _check(lib().anelm_bf16_to_f32_plus1(_ptr(dst), _ptr(src), src.numel(), _stream(stream)))


def f32_to_f16(dst, src, stream=None):
    _check(lib().anelm_f32_to_f16(_ptr(dst), _ptr(src), src.numel(), _stream(stream)))


def f16_to_f32(dst, src, stream=None):
    _check(lib().anelm_f16_to_f32(_ptr(dst), _ptr(src), src.numel(), _stream(stream)))


def softmax_workspace_size(rows, n) -> int:
    return lib().anelm_softmax_workspace_size(rows, n)


def softmax(x, workspace, stream=None):
    rows, n, ld = _rows(x)
    _check(lib().anelm_softmax(_ptr(x), rows, n, ld, _ptr(workspace), workspace.numel() * workspace.element_size(),
                               _stream(stream)))


def sample_workspace_size(rows, vocab) -> int:
    return lib().anelm_sample_workspace_size(rows, vocab)


def sample(ids, probs, logits, hist, hist_len, params: SamplingParams, r, workspace, stream=None):
    rows, vocab, ldl = _rows(logits)
    ldp = _ld(probs) if probs is not None else 0
    hist_ld = _ld(hist) if hist is not None and hist.numel() else 0
    _check(lib().anelm_sample(_ptr(ids), _ptr(probs), ldp, _ptr(logits), ldl, rows, vocab,
                              _ptr(hist) if hist_ld else None, hist_ld, _ptr(hist_len), ctypes.byref(params),
                              _ptr(r), _ptr(workspace), workspace.numel() * workspace.element_size(),
                              _stream(stream)))


def layer_ops(x, xn_in, xn_post, attn, mlp, q, k, h, g, u, w_in, w_post, wq, wk, pos, cos_tab, sin_tab, theta=1e6,
              eps=1e-6, nq=None, nk=None, stream=None):
    """The layer's five ops in one launch (anelm_layer_ops): contiguous rows,
    q [T, nq*128], k [T, nk*128], gammas of one dtype."""
    T, H = x.shape
    nq = nq if nq is not None else q.shape[1] // 128
    nk = nk if nk is not None else k.shape[1] // 128
    _check(lib().anelm_layer_ops(_ptr(x), _ptr(xn_in), _ptr(xn_post), _ptr(attn), _ptr(mlp), _ptr(q), _ptr(k), _ptr(h),
                                 _ptr(g), _ptr(u), _ptr(w_in), _ptr(w_post), _ptr(wq), _ptr(wk), _dtype_code(w_in),
                                 _ptr(pos), _ptr(cos_tab), _ptr(sin_tab), cos_tab.shape[0], theta, T, H, nq, nk,
                                 g.shape[1], eps, _stream(stream)))


def sample_noalloc(ids, probs, logits, hist, hist_len, params: SamplingParams, r, stream=None):
    """anelm_sample without a workspace: the library's static per-GPU scratch
    (4 MiB) serves instead; calls that overlap on one GPU race."""
    rows, vocab, ldl = _rows(logits)
    ldp = _ld(probs) if probs is not None else 0
    hist_ld = _ld(hist) if hist is not None and hist.numel() else 0
    _check(lib().anelm_sample_noalloc(_ptr(ids), _ptr(probs), ldp, _ptr(logits), ldl, rows, vocab,
                                      _ptr(hist) if hist_ld else None, hist_ld, _ptr(hist_len), ctypes.byref(params),
                                      _ptr(r), _stream(stream)))


def gqa_workspace_size(batch, n_heads, n_kv_heads, head_dim, capacity) -> int:
    return lib().anelm_gqa_workspace_size(batch, n_heads, n_kv_heads, head_dim, capacity)


def _nbytes(t):
    return 0 if t is None else t.numel() * t.element_size()


def gqa_attention(out, q, k_cache, v_cache, ring_start, ring_len, n_heads, n_kv_heads, head_dim, workspace,
                  q_head_stride=None, stream=None):
    """Batched decode attention.  q: [B, >= (n_heads-1)*q_head_stride + head_dim];
    out: [B, >= n_heads*head_dim], fp32 or (int16/float16) fp16; caches: [B,
    capacity, n_kv_heads*head_dim] (any per-sequence stride); ring_start /
    ring_len: int32 [B]."""
    B = q.shape[0]
    cap = k_cache.shape[1]
    _need(k_cache.stride() == v_cache.stride() and k_cache.stride(2) == 1 and k_cache.stride(1) == n_kv_heads * head_dim,
          "gqa_attention: cache layout")
    fn = lib().anelm_gqa_attention_f16 if out.element_size() == 2 else lib().anelm_gqa_attention   # fp16 output
    _check(fn(_ptr(out), _ptr(q), _ptr(k_cache), _ptr(v_cache), _ptr(ring_start), _ptr(ring_len), B, n_heads,
              n_kv_heads, head_dim, _ld(q), head_dim if q_head_stride is None else q_head_stride, _ld(out), cap,
              k_cache.stride(0), _ptr(workspace), _nbytes(workspace), _stream(stream)))


def gqa_attention_bounded(out, q, k_cache, v_cache, ring_start, ring_len, n_heads, n_kv_heads, head_dim, len_bound,
                          workspace, q_head_stride=None, stream=None):
    """gqa_attention when every ring length is known to be <= len_bound."""
    B = q.shape[0]
    cap = k_cache.shape[1]
    _need(k_cache.stride() == v_cache.stride() and k_cache.stride(2) == 1 and k_cache.stride(1) == n_kv_heads * head_dim,
          "gqa_attention: cache layout")
    _check(lib().anelm_gqa_attention_bounded(_ptr(out), _ptr(q), _ptr(k_cache), _ptr(v_cache), _ptr(ring_start),
                                             _ptr(ring_len), B, n_heads, n_kv_heads, head_dim, _ld(q),
                                             head_dim if q_head_stride is None else q_head_stride, _ld(out), cap,
                                             k_cache.stride(0), len_bound, _ptr(workspace), _nbytes(workspace),
                                             _stream(stream)))


def gqa_attention_ring(out, q, k_cache, v_cache, n_heads, n_kv_heads, head_dim, cache_start, cache_len, workspace,
                       q_head_stride=None, stream=None):
    """The reference's single-sequence form (core/cpu_ops.cpp:173-240) with
    host ring state; caches [capacity, n_kv_heads*head_dim]."""
    cap = k_cache.shape[0]
    _check(lib().anelm_gqa_attention_ring(_ptr(out), _ptr(q), _ptr(k_cache), _ptr(v_cache), n_heads, n_kv_heads,
                                          head_dim, head_dim if q_head_stride is None else q_head_stride,
                                          cache_start, cache_len, cap, _ptr(workspace), _nbytes(workspace),
                                          _stream(stream)))


def kv_ring_append(k_cache, v_cache, ring_start, ring_len, k, v, stream=None):
    """Append row b of k, v ([B, n_kv_heads*head_dim]) to sequence b's ring
    (caches [B, capacity, n_kv_heads*head_dim]) and advance its state."""
    B, cap, row = k_cache.shape
    _need(k.shape[1] == row and v.shape[1] == row and k_cache.stride() == v_cache.stride(), "kv_ring_append: shapes")
    _check(lib().anelm_kv_ring_append(_ptr(k_cache), _ptr(v_cache), _ptr(ring_start), _ptr(ring_len), _ptr(k),
                                      _ptr(v), _ld(k), _ld(v), B, 1, row, cap, k_cache.stride(0), _stream(stream)))


def kv_ring_advance(ring_start, ring_len, capacity, batch=None, stream=None):
    """Advance rings by one row each (state only).  ring_start / ring_len:
    int32 [B] or [groups, >= B] (row stride = group stride)."""
    _need(ring_start.shape == ring_len.shape and ring_start.stride() == ring_len.stride(), "kv_ring_advance: shapes")
    if ring_start.dim() == 1:
        groups, gstride, B = 1, ring_start.shape[0], ring_start.shape[0]
    else:
        groups, gstride, B = ring_start.shape[0], ring_start.stride(0), ring_start.shape[1]
    B = B if batch is None else batch
    _check(lib().anelm_kv_ring_advance(_ptr(ring_start), _ptr(ring_len), B, groups, gstride, capacity,
                                       _stream(stream)))


def gqa_attention_qk(out, q, k, v, wq, wk, pos, cos_tab, sin_tab, k_cache, v_cache, ring_start, ring_len, n_heads,
                     n_kv_heads, workspace, theta=1e6, eps=1e-6, stream=None, tiled=False, advance=False):
    """qknorm_rope_append + gqa_attention in one launch (head_dim 128) for rings
    already advanced by kv_ring_advance (advance=True: the call advances them
    first, anelm_gqa_attention_qk_append).  q: [B, >= n_heads*128], k, v: [B, >=
    n_kv_heads*128] (row slices of the qkv projection allowed, left as they
    are); out fp32 or fp16 (tiled: fp16 in the tiled layout of proj_tile_f16,
    n_heads*128 columns); caches [B, capacity, n_kv_heads*128]."""
    B = q.shape[0]
    cap = k_cache.shape[1]
    _need(k_cache.stride() == v_cache.stride() and k_cache.stride(2) == 1 and k_cache.stride(1) == n_kv_heads * 128,
          "gqa_attention_qk: cache layout")
    wdt = _dtype_code(wq if wq is not None else (wk if wk is not None else q))
    tab_len = cos_tab.shape[0] if cos_tab is not None else 0
    mode = 2 if tiled else int(out.element_size() == 2)
    fn = lib().anelm_gqa_attention_qk_append if advance else lib().anelm_gqa_attention_qk
    _check(fn(_ptr(out), mode, _ptr(q), _ptr(k), _ptr(v), _ld(q), _ld(k), _ld(v), _ptr(wq), _ptr(wk), wdt, _ptr(pos),
              _ptr(cos_tab), _ptr(sin_tab), tab_len, theta, eps, _ptr(k_cache), _ptr(v_cache), _ptr(ring_start),
              _ptr(ring_len), B, n_heads, n_kv_heads, n_heads * 128 if tiled else _ld(out), cap, k_cache.stride(0),
              _ptr(workspace), _nbytes(workspace), _stream(stream)))


def rmsnorm_gated(out, x, z, w, eps=1e-6, heads=1, stream=None):
    """x, z, out: [rows, >= heads*dim] (row slices allowed); w: [dim]."""
    rows, span, ldx = _rows(x)
    _, _, ldz = _rows(z)
    _, _, ldo = _rows(out)
    dim = w.shape[0]
    _need(span >= heads * dim, "rmsnorm_gated: row shorter than heads*dim")
    _check(lib().anelm_rmsnorm_gated(_ptr(out), _ptr(x), _ptr(z), _ptr(w), _dtype_code(w), rows, heads, dim, ldx, ldz,
                                     ldo, eps, _stream(stream)))


def l2_normalize(x, scale=1.0, heads=1, stream=None):
    """x: [rows, >= heads*dim] with dim = x.shape[1] // heads (row slices allowed)."""
    rows, span, ld = _rows(x)
    _check(lib().anelm_l2_normalize(_ptr(x), rows, heads, span // heads, ld, scale, _stream(stream)))


def conv1d_update(y, conv_state, state_pos, x, w, stream=None):
    """y, x: [B, channels]; conv_state: [B, channels, K-1]; state_pos: int32 [B]; w: [channels, K]."""
    B, ch, sl = conv_state.shape
    _need(w.shape == (ch, sl + 1) and w.is_contiguous() and conv_state.stride(2) == 1 and conv_state.stride(1) == sl,
          "conv1d_update: shapes")
    _check(lib().anelm_conv1d_update(_ptr(y), _ptr(conv_state), _ptr(state_pos), _ptr(x), _ptr(w), B, ch, sl + 1,
                                     _ld(x), _ld(y), conv_state.stride(0), _stream(stream)))


def ssm_step(y, state, q, k, v, decay, beta, n_key_heads, stream=None):
    """state: [B, n_heads, key_dim, value_dim]; q, k: [B, n_key_heads*key_dim];
    v, y: [B, n_heads*value_dim]; decay, beta: [B, n_heads]."""
    B, nh, kd, vd = state.shape
    _need(state.stride(3) == 1 and state.stride(2) == vd and state.stride(1) == kd * vd, "ssm_step: state layout")
    _need(q.stride() == k.stride() and decay.is_contiguous() and beta.is_contiguous(), "ssm_step: layouts")
    _check(lib().anelm_ssm_step(_ptr(y), _ptr(state), _ptr(q), _ptr(k), _ptr(v), _ptr(decay), _ptr(beta), B, nh,
                                n_key_heads, kd, vd, _ld(q), _ld(v), _ld(y), state.stride(0), _stream(stream)))


def ssm_step_gated_norm(out, state, q, k, v, decay, beta, z, norm_w, n_key_heads, eps=1e-6, stream=None):
    """ssm_step, then rmsnorm_gated of each head's y with gate z and weight
    norm_w ([value_dim]); out, z: [B, n_heads*value_dim]."""
    B, nh, kd, vd = state.shape
    _need(state.stride(3) == 1 and state.stride(2) == vd and state.stride(1) == kd * vd, "ssm_step: state layout")
    _need(q.stride() == k.stride() and decay.is_contiguous() and beta.is_contiguous(), "ssm_step: layouts")
    _check(lib().anelm_ssm_step_gated_norm(_ptr(out), _ptr(state), _ptr(q), _ptr(k), _ptr(v), _ptr(decay), _ptr(beta),
                                           _ptr(z), _ptr(norm_w), _dtype_code(norm_w), B, nh, n_key_heads, kd, vd, _ld(q),
                                           _ld(v), _ld(z), _ld(out), state.stride(0), eps, _stream(stream)))


def conv1d_silu_l2norm(y, conv_state, state_pos, x, w, n_key_heads, q_scale, stream=None):
    """conv1d_update (kernel size 4), SiLU and the q/k L2 normalisation of the
    decode step; channels [q heads | k heads | v], key heads of 128."""
    B, ch, sl = conv_state.shape
    _need(sl == 3 and w.shape == (ch, 4) and w.is_contiguous() and conv_state.stride(2) == 1 and
          conv_state.stride(1) == sl, "conv1d_silu_l2norm: shapes")
    _check(lib().anelm_conv1d_silu_l2norm(_ptr(y), _ptr(conv_state), _ptr(state_pos), _ptr(x), _ptr(w), B, ch,
                                          n_key_heads, _ld(x), _ld(y), conv_state.stride(0), q_scale, _stream(stream)))


def conv_ssm_step_gated_norm(out, state, conv_state, head_pos, x, conv_w, decay, beta, z, norm_w, q_scale, eps=1e-6,
                             stream=None):
    """conv1d_silu_l2norm then ssm_step_gated_norm in one launch, key and value
    heads of 128, as many key heads as value heads; head_pos: the ring
    position per (sequence, head), int32 [B, n_heads]."""
    B, nh, kd, vd = state.shape
    ch = conv_state.shape[1]
    _need(kd == 128 and vd == 128 and ch == 3 * nh * 128, "conv_ssm_step_gated_norm: heads of 128, channels")
    _need(state.stride(3) == 1 and state.stride(2) == vd and state.stride(1) == kd * vd, "ssm_step: state layout")
    _need(conv_state.shape == (B, ch, 3) and conv_state.stride(2) == 1 and conv_state.stride(1) == 3 and
          conv_w.shape == (ch, 4) and conv_w.is_contiguous(), "conv_ssm_step_gated_norm: conv shapes")
    _need(head_pos.numel() == B * nh and head_pos.is_contiguous() and str(head_pos.dtype) == "torch.int32" and
          decay.is_contiguous() and beta.is_contiguous(), "conv_ssm_step_gated_norm: layouts")
    _check(lib().anelm_conv_ssm_step_gated_norm(_ptr(out), _ptr(state), _ptr(conv_state), _ptr(head_pos), _ptr(x),
                                                _ptr(conv_w), _ptr(decay), _ptr(beta), _ptr(z), _ptr(norm_w),
                                                _dtype_code(norm_w), B, nh, _ld(x), _ld(z), _ld(out), state.stride(0),
                                                conv_state.stride(0), q_scale, eps, _stream(stream)))


def matvec(y, W, x, stream=None):
    out_dim, in_dim = W.shape
    _need(W.is_contiguous() and x.is_contiguous() and y.numel() >= out_dim, "matvec: shapes")
    _check(lib().anelm_matvec(_ptr(y), _ptr(W), _ptr(x), out_dim, in_dim, _stream(stream)))


ST_F64, ST_I32, ST_I64, ST_U8, ST_UNKNOWN = 3, 4, 5, 6, -1


class SafeTensorsFile:
    """A safetensors file opened by the library (core/safetensors.cpp:193-244).
    info(i) -> (name, dtype code, shape, offset, nbytes); load(i, dst, dtype)
    copies tensor i into device tensor dst (widened / converted on the device)."""

    def __init__(self, path):
        self._h = lib().anelm_st_open(os.fsencode(path))
        if not self._h:
            raise AnelmError(ERR_INVALID, last_error())

    def close(self):
        if self._h:
            lib().anelm_st_close(self._h)
            self._h = None

    def __enter__(self):
        return self

    def __exit__(self, *a):
        self.close()

    def __len__(self):
        return lib().anelm_st_count(self._h)

    # names are the raw bytes between the header's quotes (not necessarily
    # UTF-8); surrogateescape carries any byte through str and back
    def find(self, name):
        return lib().anelm_st_find(self._h, name.encode("utf-8", "surrogateescape"))

    def info(self, i):
        name, dt, nd = ctypes.c_char_p(), _I(), _I()
        shape = (ctypes.c_int64 * 8)()
        off, nb = ctypes.c_uint64(), ctypes.c_uint64()
        _check(lib().anelm_st_info(self._h, i, ctypes.byref(name), ctypes.byref(dt), ctypes.byref(nd), shape,
                                   ctypes.byref(off), ctypes.byref(nb)))
        return name.value.decode("utf-8", "surrogateescape"), dt.value, tuple(shape[:nd.value]), off.value, nb.value

    def host_data(self, i):
        return lib().anelm_st_host_data(self._h, i)

    def load(self, i, dst, dtype, stream=None):
        _check(lib().anelm_st_load(self._h, i, _ptr(dst), dtype, _stream(stream)))

    def load_norm(self, i, dst, expected_numel, stream=None):
        """SafeTensors::load_norm_weight: BF16 tensor i as fp32 (1+w)."""
        _check(lib().anelm_st_load_norm(self._h, i, _ptr(dst), expected_numel, _stream(stream)))


def ane_blob_header(num_elements) -> bytes:
    buf = (ctypes.c_uint8 * 128)()
    lib().anelm_ane_blob_header(buf, num_elements)
    return bytes(buf)


def write_ane_blobs(safetensors_path, output_dir, stream=None) -> int:
    n = lib().anelm_write_ane_blobs(os.fsencode(safetensors_path), os.fsencode(output_dir), _stream(stream))
    if n < 0:
        raise AnelmError(n, last_error())
    return n


class Qwen3Config(ctypes.Structure):
    _fields_ = [("hidden", ctypes.c_int), ("layers", ctypes.c_int), ("n_q_heads", ctypes.c_int),
                ("n_kv_heads", ctypes.c_int), ("head_dim", ctypes.c_int), ("intermediate", ctypes.c_int),
                ("vocab", ctypes.c_int), ("rope_theta", ctypes.c_float), ("rms_eps", ctypes.c_float)]


def linear_f16(y16, x16, w16, stream=None):
    """y16 [B, out] = fp16(x16 [B, in] . w16 [out, in]^T), fp32 accumulation."""
    batch, in_dim = x16.shape
    out_dim = w16.shape[0]
    _check(lib().anelm_linear_f16(_ptr(y16), _ptr(x16), _ptr(w16), batch, out_dim, in_dim, _ld(x16), _ld(y16),
                                  _stream(stream)))


def proj_f16(y, x, w16, stream=None):
    """y [B, out] fp32 = fp16(fp16(x) [B, in] . w16 [out, in]^T)."""
    batch, in_dim = x.shape
    out_dim = w16.shape[0]
    _check(lib().anelm_proj_f16(_ptr(y), _ptr(x), _ptr(w16), batch, out_dim, in_dim, _ld(x), _ld(y),
                                _stream(stream)))


def proj_f16_x16(y, x16, w16, stream=None):
    """proj_f16 with x16 [B, in] already rounded to fp16 (int16 or float16 tensor)."""
    batch, in_dim = x16.shape
    out_dim = w16.shape[0]
    _check(lib().anelm_proj_f16_x16(_ptr(y), _ptr(x16), _ptr(w16), batch, out_dim, in_dim, _ld(x16), _ld(y),
                                    _stream(stream)))


PROJ_STORE, PROJ_ADD, PROJ_SWIGLU, PROJ_SWIGLU_F16, PROJ_STORE_F16 = 0, 1, 2, 3, 4


def proj_f16_fused(y, x, w16, norm=None, eps=1e-6, epilogue=PROJ_STORE, stream=None):
    """Decode projection with an optional RMSNorm prologue (norm:
    bf16 gamma as int16/bfloat16 tensor) and a store / residual-add / SwiGLU
    epilogue; for SwiGLU w16 holds the gate rows then the up rows; y fp32, or
    fp16 bits (int16/float16 tensor) with PROJ_SWIGLU_F16."""
    batch, in_dim = x.shape
    out_dim = w16.shape[0] // 2 if epilogue in (PROJ_SWIGLU, PROJ_SWIGLU_F16) else w16.shape[0]
    _check(lib().anelm_proj_f16_fused(_ptr(y), _ptr(x), _ptr(w16), batch, out_dim, in_dim, _ld(x), _ld(y),
                                      _ptr(norm), eps, epilogue, _stream(stream)))


def proj_f16_x16_fused(y, x16, w16, epilogue=PROJ_STORE, stream=None):
    """The fused epilogues on fp16 rows x16 (int16/float16 tensor of fp16
    bits); y fp32, or fp16 bits with PROJ_SWIGLU_F16."""
    batch, in_dim = x16.shape
    out_dim = w16.shape[0] // 2 if epilogue in (PROJ_SWIGLU, PROJ_SWIGLU_F16) else w16.shape[0]
    _check(lib().anelm_proj_f16_x16_fused(_ptr(y), _ptr(x16), _ptr(w16), batch, out_dim, in_dim, _ld(x16), _ld(y),
                                          epilogue, _stream(stream)))


def proj_tiled_size(out_dim, in_dim):
    """Bytes of the tiled copy of an [out_dim, in_dim] fp16 W (0 if in_dim % 32)."""
    return lib().anelm_proj_tiled_size(out_dim, in_dim)


def proj_tile_f16(w_tiled, w16, stream=None):
    """w_tiled (uint8/int16 tensor of proj_tiled_size bytes) = the tiled layout of w16 [out, in]."""
    out_dim, in_dim = w16.shape
    _check(lib().anelm_proj_tile_f16(_ptr(w_tiled), _ptr(w16), out_dim, in_dim, _stream(stream)))


def proj_f16_x16_tiled(y, x16, w_tiled, out_dim, epilogue=PROJ_STORE, stream=None):
    """The fused epilogues of proj_f16_x16_fused on a tiled W (proj_tile_f16),
    plus PROJ_STORE_F16: y [B, out_dim] fp32, or fp16 bits with PROJ_STORE_F16 /
    PROJ_SWIGLU_F16; for the SwiGLU the tiled W holds 2*out_dim rows."""
    batch, in_dim = x16.shape
    _check(lib().anelm_proj_f16_x16_tiled(_ptr(y), _ptr(x16), _ptr(w_tiled), batch, out_dim, in_dim, _ld(x16),
                                          _ld(y), epilogue, _stream(stream)))


PROJ_SWIGLU_F16_TILED = 5


def proj_f16_tt(y, x_t, w_t, batch, out_dim, in_dim, epilogue=PROJ_STORE, stream=None):
    """The tiled-W projection on x_t in the tiled layout too (batch rows, in_dim
    columns); y [batch, out_dim] fp32 / fp16 bits, or with PROJ_SWIGLU_F16_TILED
    fp16 in the tiled layout (batch rows, out_dim columns)."""
    ld_y = out_dim if epilogue == PROJ_SWIGLU_F16_TILED else _ld(y)
    _check(lib().anelm_proj_f16_tt(_ptr(y), _ptr(x_t), _ptr(w_t), batch, out_dim, in_dim, ld_y, epilogue,
                                   _stream(stream)))


class Qwen3Model:
    """A Qwen3 checkpoint in HBM with per-sequence KV rings (anelm_qwen3_*)."""

    def __init__(self, path, cfg: Qwen3Config, max_batch: int, kv_capacity: int = 2048, stream=None):
        self.cfg = cfg
        self._h = lib().anelm_qwen3_load(os.fsencode(path), ctypes.byref(cfg), max_batch, kv_capacity,
                                         _stream(stream))
        if not self._h:
            raise AnelmError(ERR_INVALID, last_error())

    def reset(self, stream=None):
        _check(lib().anelm_qwen3_reset(self._h, _stream(stream)))

    def forward(self, ids, pos, logits, bad_ids=None, stream=None):
        _check(lib().anelm_qwen3_forward(self._h, _ptr(ids), _ptr(pos), ids.shape[0], _ptr(logits), _ld(logits),
                                         _ptr(bad_ids), _stream(stream)))

    def close(self):
        if getattr(self, "_h", None):
            lib().anelm_qwen3_free(self._h)
            self._h = None

    def __del__(self):
        try:
            if getattr(self, "_h", None) and _lib is not None:
                _lib.anelm_qwen3_free(self._h)
        except Exception:   # interpreter shutdown
            pass
        self._h = None
