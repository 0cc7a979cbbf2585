"""RMSNorm (core/cpu_ops.cpp:25-31), fused add+RMSNorm (qwen3.cpp:516-518),
q/k-norm + RoPE (qwen3.cpp:444-472), apply_rope_cached (cpu_ops.cpp:56-80)
and the RoPE table (qwen3.cpp:200-219) on the GPU against the oracle.
Tolerance: max relative error <= 1e-5 (RoPE: relative to |a c| + |b s|)."""
import numpy as np
import pytest

from helpers import REL_TOL, assert_bitexact, dev, gamma_f16, host, max_rel_err, rope_den

pytestmark = pytest.mark.gpu
THETA = 1e6
EPS = 1e-6


def _gamma(rng, n, dt):
    import torch

    g16 = gamma_f16(rng, n)
    w32 = g16.view(np.float16).astype(np.float32)          # exact widening: the oracle's gamma
    if dt == "f16":
        return dev(g16).view(torch.float16), w32
    if dt == "bf16":
        wb = (w32.view(np.uint32) >> 16).astype(np.uint16)
        return dev(wb).view(torch.bfloat16), (wb.astype(np.uint32) << 16).view(np.float32)
    return dev(w32), w32


@pytest.mark.parametrize("rows,dim", [(1, 1024), (2048, 1024), (64, 2560), (512, 4096), (3, 1000), (5, 7),
                                      (2, 5120), (2, 8192), (4, 12288)])
@pytest.mark.parametrize("dt", ["f16", "f32", "bf16"])
def test_rmsnorm(hip, orc, rng, rows, dim, dt):
    import torch

    x = rng.standard_normal((rows, dim), dtype=np.float32)
    wt, w32 = _gamma(rng, dim, dt)
    out = torch.empty(rows, dim, device="cuda")
    hip.rmsnorm(out, dev(x), wt, EPS)
    assert max_rel_err(host(out), orc.rmsnorm_rows(x, w32, EPS)) <= REL_TOL


@pytest.mark.parametrize("rows,dim", [(1, 1024), (64, 1024), (64, 2560), (3, 1000), (5, 7), (2, 8192)])
@pytest.mark.parametrize("dt", ["f16", "bf16"])
def test_rmsnorm_f16_output(hip, orc, rng, rows, dim, dt):
    """The fp16-output RMSNorm: bit-identical to the fp32 RMSNorm followed by
    the RNE narrowing (same kernel layout, dim a multiple of 4) and within one
    fp16 ulp (plus the norm's tolerance) of the oracle's RMSNorm rounded."""
    import torch

    x = (3 * rng.standard_normal((rows, dim))).astype(np.float32)
    wt, w32 = _gamma(rng, dim, dt)
    out16 = torch.empty(rows, dim, dtype=torch.int16, device="cuda")
    hip.rmsnorm_f16(out16, dev(x), wt, EPS)
    got = host(out16).view(np.float16).astype(np.float64)
    if dim % 4 == 0:
        ref32 = torch.empty(rows, dim, device="cuda")
        hip.rmsnorm(ref32, dev(x), wt, EPS)
        ref16 = torch.empty(rows, dim, dtype=torch.int16, device="cuda")
        hip.f32_to_f16(ref16, ref32)
        assert_bitexact(host(out16), host(ref16), "rmsnorm_f16 vs rmsnorm + narrow")
    want = orc.rmsnorm_rows(x, w32, EPS).astype(np.float64)
    ulp = np.spacing(np.abs(want).astype(np.float16)).astype(np.float64)
    assert np.all(np.abs(got - want) <= ulp + np.abs(want) * REL_TOL)


def test_rmsnorm_f16_gamma_every_pattern(hip, orc):
    """The row RMSNorm's fp16 gamma widened for all 65,536 bit patterns, four
    calls of 16,384 columns (the row kernel's full-row shape): x is all ones,
    so every column's x*s is the same float s (the sum of squares is exact),
    and each output is fl(s * gamma).  Non-NaN gammas (normal, subnormal,
    zero, infinity: the conversion instruction) must match the oracle's exact
    widening bit for bit; the waves that hold NaN patterns take the integer
    widening and give NaN."""
    import torch

    x = np.ones((2, 16384), np.float32)
    for k in range(4):
        bits = np.arange(k * 16384, (k + 1) * 16384, dtype=np.uint32).astype(np.uint16)
        w16 = bits.view(np.float16)
        out = torch.empty(2, 16384, device="cuda")
        hip.rmsnorm(out, dev(x), dev(bits).view(torch.float16), 1e-6)
        got = host(out)
        want = orc.rmsnorm(x[0], w16.astype(np.float32), 1e-6)   # numpy's fp16 widening is exact
        nan = np.isnan(w16)
        for r in range(2):
            assert_bitexact(got[r][~nan], want[~nan], f"patterns {k * 16384}..: row {r}")
            assert np.all(np.isnan(got[r][nan]))


def test_rmsnorm_in_place_and_strided(hip, orc, rng):
    import torch

    x = rng.standard_normal((33, 1536), dtype=np.float32)
    wt, w32 = _gamma(rng, 1024, "f16")
    t = dev(x)
    view = t[:, 256:1280]                       # rows of 1024 at stride 1536
    hip.rmsnorm(view, view, wt, EPS)            # out aliases x (qwen3.cpp:530)
    got = host(t)
    assert max_rel_err(got[:, 256:1280], orc.rmsnorm_rows(x[:, 256:1280], w32, EPS)) <= REL_TOL
    assert np.array_equal(got[:, :256], x[:, :256]) and np.array_equal(got[:, 1280:], x[:, 1280:])


@pytest.mark.parametrize("rows,dim", [(1, 1024), (2048, 1024), (64, 2560), (256, 4096), (3, 1001)])
def test_add_rmsnorm(hip, orc, rng, rows, dim):
    import torch

    x = rng.standard_normal((rows, dim), dtype=np.float32)
    y = rng.standard_normal((rows, dim), dtype=np.float32)
    wt, w32 = _gamma(rng, dim, "f16")
    xt, out = dev(x), torch.empty(rows, dim, device="cuda")
    hip.add_rmsnorm(xt, dev(y), out, wt, EPS)
    assert_bitexact(host(xt), x + y, "residual stream")
    assert max_rel_err(host(out), orc.rmsnorm_rows(x + y, w32, EPS)) <= REL_TOL


def test_add_rmsnorm_y_aliases_out(hip, orc, rng):
    """attn_out lives in x_norm_ (qwen3.cpp:508-518): y == out."""
    x = rng.standard_normal((16, 1024), dtype=np.float32)
    y = rng.standard_normal((16, 1024), dtype=np.float32)
    wt, w32 = _gamma(rng, 1024, "f32")
    xt, yt = dev(x), dev(y)
    hip.add_rmsnorm(xt, yt, yt, wt, EPS)
    assert_bitexact(host(xt), x + y, "residual stream")
    assert max_rel_err(host(yt), orc.rmsnorm_rows(x + y, w32, EPS)) <= REL_TOL


def _check_qk(orc, q, k, q2, k2, wq32, wk32, pos, c_tab, s_tab, nq, nk, D):
    """Compare GPU q2/k2 with the oracle; errors scaled by |a c| + |b s|."""
    T = len(pos)
    rq, rk = orc.qknorm_rope(q, k, wq32, wk32, pos, c_tab, s_tab, THETA, nq, nk, D)
    nq0, nk0 = orc.qknorm_rope(q, k, wq32, wk32, np.zeros(T, np.int32), c_tab, s_tab, THETA, nq, nk, D)
    half = D // 2
    inv = orc.rope_inv_freq(D, THETA)
    ang = (pos.astype(np.float32)[:, None] * inv[None, :]).astype(np.float64)
    c, s = np.cos(ang)[:, None, :], np.sin(ang)[:, None, :]
    for got, ref, n0, nh, ld in ((q2, rq, nq0, nq, q.shape[1]), (k2, rk, nk0, nk, k.shape[1])):
        if nh == 0:
            continue
        g = got[:, :nh * D].reshape(T, nh, D)
        r = ref[:, :nh * D].reshape(T, nh, D)
        den = rope_den(n0[:, :nh * D].reshape(T, nh, D), c, s, half)
        assert max_rel_err(g, r, den) <= REL_TOL
        assert np.array_equal(got[:, nh * D:], ref[:, nh * D:])   # bytes past the heads untouched


@pytest.mark.parametrize("T,nq,nk,pmax,tab", [(1, 16, 8, 4096, 16384),       # 0.6B decode
                                              (256, 16, 8, 2048, 16384),     # 0.6B prefill rows
                                              (64, 32, 8, 32768, 16384),     # 4B batched decode: half fallback
                                              (128, 32, 8, 8192, 16384),     # 8B prefill rows
                                              (7, 5, 3, 100, 0)])            # no table at all
def test_qknorm_rope(hip, orc, rng, T, nq, nk, pmax, tab):
    import torch

    D = 128
    q = rng.standard_normal((T, nq * D), dtype=np.float32)
    k = rng.standard_normal((T, nk * D), dtype=np.float32)
    pos = rng.integers(0, pmax, T).astype(np.int32)
    pos[0] = 0
    if T > 2:
        pos[1] = pmax - 1
    wq, wq32 = _gamma(rng, D, "f16")
    wk, wk32 = _gamma(rng, D, "f16")
    c_tab, s_tab = orc.rope_table(tab, D, THETA) if tab else (None, None)
    qt, kt = dev(q), dev(k)
    hip.qknorm_rope(qt, kt, wq, wk, dev(pos), dev(c_tab) if tab else None, dev(s_tab) if tab else None, THETA,
                    EPS, nq=nq, nk=nk)
    _check_qk(orc, q, k, host(qt), host(kt), wq32, wk32, pos, c_tab, s_tab, nq, nk, D)


def test_qknorm_rope_fused_qkv_layout(hip, orc, rng):
    """q and k as slices of the fused [q|k|v] row (qwen3.cpp:440-442)."""
    T, nq, nk, D = 40, 16, 8, 128
    row = (nq + 2 * nk) * D
    qkv = rng.standard_normal((T, row), dtype=np.float32)
    pos = np.arange(T, dtype=np.int32) * 37
    wq, wq32 = _gamma(rng, D, "f32")
    wk, wk32 = _gamma(rng, D, "f32")
    c_tab, s_tab = orc.rope_table(2048, D, THETA)
    t = dev(qkv)
    hip.qknorm_rope(t[:, :nq * D], t[:, nq * D:(nq + nk) * D], wq, wk, dev(pos), dev(c_tab), dev(s_tab), THETA, EPS,
                    nq=nq, nk=nk)
    got = host(t)
    q, k = np.ascontiguousarray(qkv[:, :nq * D]), np.ascontiguousarray(qkv[:, nq * D:(nq + nk) * D])
    _check_qk(orc, q, k, np.ascontiguousarray(got[:, :nq * D]), np.ascontiguousarray(got[:, nq * D:(nq + nk) * D]),
              wq32, wk32, pos, c_tab, s_tab, nq, nk, D)
    assert np.array_equal(got[:, (nq + nk) * D:], qkv[:, (nq + nk) * D:])   # v untouched


def test_qknorm_rope_without_norm(hip, orc, rng):
    T, nq, nk, D = 9, 4, 2, 128
    q = rng.standard_normal((T, nq * D), dtype=np.float32)
    k = rng.standard_normal((T, nk * D), dtype=np.float32)
    pos = rng.integers(0, 20000, T).astype(np.int32)
    c_tab, s_tab = orc.rope_table(16384, D, THETA)
    qt, kt = dev(q), dev(k)
    hip.qknorm_rope(qt, kt, None, None, dev(pos), dev(c_tab), dev(s_tab), THETA, EPS, nq=nq, nk=nk)
    _check_qk(orc, q, k, host(qt), host(kt), None, None, pos, c_tab, s_tab, nq, nk, D)


@pytest.mark.parametrize("D", [64, 256, 96])
def test_qknorm_rope_other_head_dims(hip, orc, rng, D):
    T, nq, nk = 11, 3, 2
    q = rng.standard_normal((T, nq * D), dtype=np.float32)
    k = rng.standard_normal((T, nk * D), dtype=np.float32)
    pos = rng.integers(0, 3000, T).astype(np.int32)
    wq, wq32 = _gamma(rng, D, "f16")
    wk, wk32 = _gamma(rng, D, "f16")
    c_tab, s_tab = orc.rope_table(1024, D, THETA)
    qt, kt = dev(q), dev(k)
    hip.qknorm_rope(qt, kt, wq, wk, dev(pos), dev(c_tab), dev(s_tab), THETA, EPS, nq=nq, nk=nk, head_dim=D)
    _check_qk(orc, q, k, host(qt), host(kt), wq32, wk32, pos, c_tab, s_tab, nq, nk, D)


@pytest.mark.parametrize("with_row", [True, False])
def test_rope_cached(hip, orc, rng, with_row):
    """Qwen3.5 call shape (qwen3_5.cpp:595-597): q stride 2*head_dim, partial rotary."""
    D, rot, nq, nk, pos = 256, 64, 8, 2, 1234
    q = rng.standard_normal(nq * 2 * D, dtype=np.float32)
    k = rng.standard_normal(nk * D, dtype=np.float32)
    c_tab, s_tab = orc.rope_table(2048, rot, THETA)
    cr, sr = (c_tab[pos], s_tab[pos]) if with_row else (None, None)
    qt, kt = dev(q), dev(k)
    hip.rope_cached(qt, kt, nq, nk, D, 2 * D, D, rot, pos, THETA, dev(cr) if with_row else None,
                    dev(sr) if with_row else None)
    rq, rk = orc.rope_cached(q, k, nq, nk, D, 2 * D, D, rot, pos, THETA, cr, sr)
    gq, gk = host(qt), host(kt)
    scale = np.abs(q).max()
    assert np.max(np.abs(gq - rq)) <= 4e-6 * scale
    assert np.max(np.abs(gk - rk)) <= 4e-6 * scale
    mask = np.ones(nq * 2 * D, bool)
    for h in range(nq):
        mask[h * 2 * D:h * 2 * D + rot] = False
    assert np.array_equal(gq[mask], q[mask])


@pytest.mark.parametrize("n_pos", [16384, 32768])
def test_rope_table(hip, orc, n_pos):
    import torch

    c, s = torch.empty(n_pos, 64, device="cuda"), torch.empty(n_pos, 64, device="cuda")
    hip.rope_table(c, s, THETA)
    rc, rs = orc.rope_table(n_pos, 128, THETA)
    gc, gs = host(c), host(s)
    assert np.all(gc[0] == 1.0) and np.all(gs[0] == 0.0)
    assert np.max(np.abs(gc - rc)) <= 2.0 ** -22 and np.max(np.abs(gs - rs)) <= 2.0 ** -22


@pytest.mark.parametrize("B,nq,nk,cap,fill,dt", [(1, 16, 8, 64, 0, "bf16"), (64, 16, 8, 64, 10, "bf16"),
                                                 (5, 32, 8, 16, 16, "f16"), (3, 4, 2, 8, 40, "f32"),
                                                 (2, 64, 8, 4, 3, "bf16"), (7, 0, 4, 32, 31, "f16")])
def test_qknorm_rope_append_matches_separate_kernels(hip, orc, rng, B, nq, nk, cap, fill, dt):
    """The decode step's fused q/k norm + RoPE + ring append equals
    anelm_qknorm_rope followed by anelm_kv_ring_append bit for bit: rotated
    q/k in the fused [q|k|v] rows, cache contents and ring state, over rings
    empty, part-full, full and wrapped (fill appends before the step), with
    some positions past the table (the fallback angle)."""
    import torch

    D = 128
    row = (nq + 2 * nk) * D
    qkv = rng.standard_normal((B, row), dtype=np.float32)
    pos = rng.integers(0, 3000, B).astype(np.int32)
    wq, _ = _gamma(rng, D, dt)
    wk, _ = _gamma(rng, D, dt)
    c_tab, s_tab = orc.rope_table(2048, D, THETA)
    caches = []
    for _ in range(2):
        kc = torch.zeros(B, cap, nk * D, device="cuda")
        vc = torch.zeros(B, cap, nk * D, device="cuda")
        rs = torch.zeros(B, dtype=torch.int32, device="cuda")
        rl = torch.zeros(B, dtype=torch.int32, device="cuda")
        for f in range(fill):   # the same history in both
            kv = dev(np.full((B, 2 * nk * D), float(f + 1), np.float32))
            hip.kv_ring_append(kc, vc, rs, rl, kv[:, :nk * D], kv[:, nk * D:])
        caches.append((kc, vc, rs, rl))
    a, b = dev(qkv), dev(qkv)
    q_of = lambda t: t[:, :nq * D] if nq else None
    kc, vc, rs, rl = caches[0]
    hip.qknorm_rope(q_of(a), a[:, nq * D:(nq + nk) * D], wq, wk, dev(pos), dev(c_tab), dev(s_tab), THETA, EPS,
                    nq=nq, nk=nk)
    hip.kv_ring_append(kc, vc, rs, rl, a[:, nq * D:(nq + nk) * D], a[:, (nq + nk) * D:])
    kc2, vc2, rs2, rl2 = caches[1]
    hip.qknorm_rope_append(q_of(b) if nq else b[:, :0], b[:, nq * D:(nq + nk) * D], b[:, (nq + nk) * D:], wq, wk,
                           dev(pos), dev(c_tab), dev(s_tab), kc2, vc2, rs2, rl2, THETA, EPS, nq=nq, nk=nk)
    assert_bitexact(host(b), host(a), "q|k|v rows")
    assert_bitexact(host(kc2), host(kc), "k cache")
    assert_bitexact(host(vc2), host(vc), "v cache")
    assert np.array_equal(host(rs2), host(rs)) and np.array_equal(host(rl2), host(rl))


@pytest.mark.parametrize("B,nq,nk,cap,dt,out16", [
    (1, 16, 8, 32, "bf16", False),     # one chunk (cap <= 32): the final-output launch
    (3, 16, 8, 32, "f16", True),
    (2, 32, 8, 4096, "bf16", False),   # split launch, short and long rings
    (2, 16, 8, 4096, "f32", True),
    (5, 64, 4, 512, "bf16", False),    # 16 q heads per kv head: two launches of 8
    (4, 16, 8, 256, "f16", False),
    (64, 16, 8, 1024, "bf16", True),   # Qwen3-0.6B attention shapes at 64 sequences
])
def test_gqa_attention_qk_matches_separate_kernels(hip, orc, rng, B, nq, nk, cap, dt, out16):
    """Rings advanced once, then the fused q/k norm + RoPE + attention, equal
    anelm_qknorm_rope_append then anelm_gqa_attention bit for bit: outputs,
    both caches and ring state, over rings of random start and length (empty,
    full and wrapped among them) and positions past the RoPE table; the raw
    q|k|v rows are left unchanged."""
    import torch

    D = 128
    row = (nq + 2 * nk) * D
    qkv = rng.standard_normal((B, row), dtype=np.float32)
    pos = rng.integers(0, 3000, B).astype(np.int32)
    wq, _ = _gamma(rng, D, dt)
    wk, _ = _gamma(rng, D, dt)
    c_tab, s_tab = orc.rope_table(2048, D, THETA)
    kc0 = rng.standard_normal((B, cap, nk * D), dtype=np.float32)
    vc0 = rng.standard_normal((B, cap, nk * D), dtype=np.float32)
    rs0 = rng.integers(-cap, 2 * cap, B).astype(np.int32)
    rl0 = rng.integers(0, cap + 1, B).astype(np.int32)
    rl0[0] = cap        # a full ring that wraps on this row
    if B > 1:
        rl0[1] = 0      # an empty ring
    if B > 2:
        rl0[2] = cap - 1
    odt = torch.float16 if out16 else torch.float32
    ws = torch.zeros(max(hip.gqa_workspace_size(B, nq, nk, D, cap), 16), dtype=torch.uint8, device="cuda")
    tabs = (dev(pos), dev(c_tab), dev(s_tab))

    a = dev(qkv)
    kc, vc, rs, rl = dev(kc0), dev(vc0), dev(rs0), dev(rl0)
    hip.qknorm_rope_append(a[:, :nq * D], a[:, nq * D:(nq + nk) * D], a[:, (nq + nk) * D:], wq, wk, *tabs, kc, vc,
                           rs, rl, THETA, EPS, nq=nq, nk=nk)
    ref = torch.full((B, nq * D), float("nan"), dtype=odt, device="cuda")
    hip.gqa_attention(ref, a[:, :nq * D], kc, vc, rs, rl, nq, nk, D, ws)

    b = dev(qkv)
    kc2, vc2, rs2, rl2 = dev(kc0), dev(vc0), dev(rs0), dev(rl0)
    hip.kv_ring_advance(rs2, rl2, cap)
    got = torch.full((B, nq * D), float("nan"), dtype=odt, device="cuda")
    hip.gqa_attention_qk(got, b[:, :nq * D], b[:, nq * D:(nq + nk) * D], b[:, (nq + nk) * D:], wq, wk, *tabs, kc2,
                         vc2, rs2, rl2, nq, nk, ws, THETA, EPS)
    assert_bitexact(host(got), host(ref), "attention output")
    assert_bitexact(host(kc2), host(kc), "k cache")
    assert_bitexact(host(vc2), host(vc), "v cache")
    assert np.array_equal(host(rs2), host(rs)) and np.array_equal(host(rl2), host(rl))
    assert_bitexact(host(b), qkv, "raw q|k|v rows")

    # the same call with the advance inside it (anelm_gqa_attention_qk_append)
    kc3, vc3, rs3, rl3 = dev(kc0), dev(vc0), dev(rs0), dev(rl0)
    got3 = torch.full((B, nq * D), float("nan"), dtype=odt, device="cuda")
    hip.gqa_attention_qk(got3, b[:, :nq * D], b[:, nq * D:(nq + nk) * D], b[:, (nq + nk) * D:], wq, wk, *tabs, kc3,
                         vc3, rs3, rl3, nq, nk, ws, THETA, EPS, advance=True)
    assert_bitexact(host(got3), host(ref), "attention output (advance in the call)")
    assert_bitexact(host(kc3), host(kc), "k cache (advance in the call)")
    assert_bitexact(host(vc3), host(vc), "v cache (advance in the call)")
    assert np.array_equal(host(rs3), host(rs)) and np.array_equal(host(rl3), host(rl))


@pytest.mark.parametrize("B,cap", [(3, 64), (2, 1024)])
def test_gqa_attention_qk_append_steps(hip, orc, rng, B, cap):
    """Successive decode steps through anelm_gqa_attention_qk_append, from
    empty rings past a wrap of the smaller ring, equal anelm_qknorm_rope_append
    then anelm_gqa_attention step for step, bit for bit (outputs, caches and
    ring state), with one workspace reused by every step."""
    import torch

    D, nq, nk, dt = 128, 16, 8, "bf16"
    row = (nq + 2 * nk) * D
    wq, _ = _gamma(rng, D, dt)
    wk, _ = _gamma(rng, D, dt)
    c_tab, s_tab = orc.rope_table(2048, D, THETA)
    tabs = (dev(c_tab), dev(s_tab))
    ws = torch.zeros(max(hip.gqa_workspace_size(B, nq, nk, D, cap), 16), dtype=torch.uint8, device="cuda")
    ws2 = torch.zeros_like(ws)
    kc = torch.zeros((B, cap, nk * D), device="cuda")
    vc = torch.zeros_like(kc)
    kc2, vc2 = kc.clone(), vc.clone()
    rs = torch.zeros(B, dtype=torch.int32, device="cuda")
    rl = torch.zeros_like(rs)
    rs2, rl2 = rs.clone(), rl.clone()
    steps = cap + 5 if cap <= 64 else 70
    for t in range(steps):
        raw = rng.standard_normal((B, row), dtype=np.float32)
        pos = dev(np.full(B, t, np.int32))
        a = dev(raw)   # normalised and rotated in place by the separate kernels
        hip.qknorm_rope_append(a[:, :nq * D], a[:, nq * D:(nq + nk) * D], a[:, (nq + nk) * D:], wq, wk, pos,
                               tabs[0], tabs[1], kc, vc, rs, rl, THETA, EPS, nq=nq, nk=nk)
        ref = torch.full((B, nq * D), float("nan"), device="cuda")
        hip.gqa_attention(ref, a[:, :nq * D], kc, vc, rs, rl, nq, nk, D, ws)
        b = dev(raw)
        got = torch.full((B, nq * D), float("nan"), device="cuda")
        hip.gqa_attention_qk(got, b[:, :nq * D], b[:, nq * D:(nq + nk) * D], b[:, (nq + nk) * D:], wq, wk, pos,
                             tabs[0], tabs[1], kc2, vc2, rs2, rl2, nq, nk, ws2, THETA, EPS, advance=True)
        assert_bitexact(host(got), host(ref), f"attention output, step {t}")
    assert_bitexact(host(kc2), host(kc), "k cache")
    assert_bitexact(host(vc2), host(vc), "v cache")
    assert np.array_equal(host(rs2), host(rs)) and np.array_equal(host(rl2), host(rl))
    assert int(host(rl2).min()) == min(steps, cap)


def test_kv_ring_advance_layers(hip, rng):
    """Advancing [layers, max_batch] ring state for the first B sequences of
    every layer equals one anelm_kv_ring_append per ring (state only), and
    leaves the sequences past B alone."""
    import torch

    L, Bmax, B, cap, row = 5, 12, 9, 16, 8
    rs0 = rng.integers(-cap, 2 * cap, (L, Bmax)).astype(np.int32)
    rl0 = rng.integers(0, cap + 1, (L, Bmax)).astype(np.int32)
    rs, rl = dev(rs0), dev(rl0)
    hip.kv_ring_advance(rs, rl, cap, batch=B)
    for l in range(L):
        r_s, r_l = dev(rs0[l, :B]), dev(rl0[l, :B])
        kc = torch.zeros(B, cap, row, device="cuda")
        kv = torch.zeros(B, row, device="cuda")
        hip.kv_ring_append(kc, kc.clone(), r_s, r_l, kv, kv)
        assert np.array_equal(host(rs)[l, :B], host(r_s)) and np.array_equal(host(rl)[l, :B], host(r_l))
    assert np.array_equal(host(rs)[:, B:], rs0[:, B:]) and np.array_equal(host(rl)[:, B:], rl0[:, B:])


@pytest.mark.parametrize("dim", [1024, 4096])
@pytest.mark.parametrize("kind", ["f32", "f16", "tiled", "add", "add_inplace"])
def test_rmsnorm_many_rows_same_bits(hip, orc, rng, dim, kind):
    """8192 rows and 512 rows get the same launch geometry (the row count
    picks the lanes per row, the same from 256 rows up), so the same rows
    must come out with the same bits, whatever the grid size; and the rows
    match the oracle."""
    import torch

    rows = 8192
    x = rng.standard_normal((rows, dim), dtype=np.float32)
    y = rng.standard_normal((rows, dim), dtype=np.float32)
    wt, w32 = _gamma(rng, dim, "f16")

    def run(n):
        xs = dev(x[:n].copy())
        if kind == "f32":
            o = torch.empty(n, dim, device="cuda")
            hip.rmsnorm(o, xs, wt, EPS)
            return host(o), None
        if kind == "f16":
            o = torch.empty(n, dim, dtype=torch.int16, device="cuda")
            hip.rmsnorm_f16(o, xs, wt, EPS)
            return host(o), None
        if kind == "tiled":
            o = torch.zeros(hip.proj_tiled_size(n, dim) // 2, dtype=torch.int16, device="cuda")
            hip.rmsnorm_f16_tiled(o, xs, wt, EPS)
            return host(o), None
        ys = dev(y[:n].copy())
        if kind == "add":
            o = torch.empty(n, dim, device="cuda")
            hip.add_rmsnorm(xs, ys, o, wt, EPS)
            return host(o), host(xs)
        hip.add_rmsnorm(xs, ys, ys, wt, EPS)   # out aliases y, same pitch
        return host(ys), host(xs)

    big, big_x = run(rows)
    small, small_x = run(512)
    if kind == "tiled":
        assert_bitexact(big[: small.size], small, "tiled rmsnorm: 8192 rows vs 512")
    else:
        assert_bitexact(big[:512], small, f"{kind}: 8192 rows vs 512")
    if big_x is not None:
        assert_bitexact(big_x[:512], small_x, f"{kind}: updated x, 8192 rows vs 512")
        assert_bitexact(big_x, x + y, f"{kind}: updated x")
    if kind in ("f32", "add", "add_inplace"):
        src = x + y if kind != "f32" else x
        assert max_rel_err(big, orc.rmsnorm_rows(src, w32, EPS)) <= REL_TOL
