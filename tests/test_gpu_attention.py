"""GQA decode attention over KV rings (core/cpu_ops.cpp:173-240) and the ring
append (models/llm/qwen3.cpp:475-488) on the GPU, against the oracle on the
same inputs.  Attention outputs must be within 1e-5 relative to
sum_t p_t |v_t[d]| (the magnitude of the terms the output sums; the output
itself can cancel to ~0); the ring append is bit-exact."""
import numpy as np
import pytest

from helpers import assert_bitexact, attention_fp64, dev, host

pytestmark = pytest.mark.gpu
ATTN_TOL = 1e-5


def ring_call(hip, q, kc, vc, nq, nk, D, start, length, qs=None):
    import torch

    out = torch.full((nq, D), float("nan"), device="cuda")
    n = hip.gqa_workspace_size(1, nq, nk, D, kc.shape[0])
    ws = torch.zeros(max(n, 1), dtype=torch.uint8, device="cuda")
    hip.gqa_attention_ring(out, dev(q), dev(kc), dev(vc), nq, nk, D, start, length, ws, q_head_stride=qs)
    return host(out)


def check(got, q, kc, vc, nq, nk, D, start, length, orc, qs=None):
    ref = orc.gqa_attention(q, kc, vc, nq, nk, D, start, length, q_head_stride=qs)
    _, bound = attention_fp64(q, kc, vc, nq, nk, D, start, length, qs)
    err = np.abs(got.astype(np.float64) - ref) / np.maximum(bound, 1e-30)
    assert float(err.max()) <= ATTN_TOL, float(err.max())


@pytest.mark.parametrize("nq,nk,D,cap,start,length,qs", [
    (16, 8, 128, 2048, 0, 1, None),          # one position
    (16, 8, 128, 2048, 2047, 2, None),       # wraps right away
    (32, 8, 128, 2048, 1500, 2048, None),    # full ring, 8B shapes
    (32, 8, 128, 2048, 3, 700, 256),         # q head stride 2*head_dim
    (40, 8, 128, 512, 100, 500, None),       # groups of 5
    (64, 8, 128, 256, 200, 256, None),       # groups of 8
    (16, 2, 256, 300, 290, 299, None),       # head_dim 256, groups of 8 in two passes
    (8, 8, 64, 100, 50, 77, None),           # head_dim 64, no sharing
    (16, 1, 64, 4096, 4000, 4096, None),     # one kv head, long ring
])
def test_ring_form_matches_oracle(hip, orc, rng, nq, nk, D, cap, start, length, qs):
    qsz = (nq - 1) * (qs or D) + D
    q = rng.standard_normal(qsz).astype(np.float32)
    kc = rng.standard_normal((cap, nk * D)).astype(np.float32)
    vc = rng.standard_normal((cap, nk * D)).astype(np.float32)
    got = ring_call(hip, q, kc, vc, nq, nk, D, start, length, qs)
    check(got, q, kc, vc, nq, nk, D, start, length, orc, qs)


def test_empty_and_single(hip, rng):
    nq, nk, D, cap = 32, 8, 128, 64
    q = rng.standard_normal(nq * D).astype(np.float32)
    kc = rng.standard_normal((cap, nk * D)).astype(np.float32)
    vc = rng.standard_normal((cap, nk * D)).astype(np.float32)
    assert np.array_equal(ring_call(hip, q, kc, vc, nq, nk, D, 5, 0), np.zeros((nq, D), np.float32))
    assert np.array_equal(ring_call(hip, q, kc, vc, nq, nk, D, 5, -4), np.zeros((nq, D), np.float32))
    one = ring_call(hip, q, kc, vc, nq, nk, D, 9, 1)   # p = 1 exactly: out = v
    for h in range(nq):
        assert np.array_equal(one[h], vc[9].reshape(nk, D)[h // 4])


def test_peaked_and_uniform_scores(hip, orc, rng):
    """A dominant key (weights underflow to 0 elsewhere) and identical keys
    (all weights equal), the two extremes of the softmax."""
    nq, nk, D, cap = 8, 2, 128, 1024
    kc = np.tile(rng.standard_normal(nk * D).astype(np.float32), (cap, 1))
    vc = rng.standard_normal((cap, nk * D)).astype(np.float32)
    q = rng.standard_normal(nq * D).astype(np.float32)
    check(ring_call(hip, q, kc, vc, nq, nk, D, 77, 1000), q, kc, vc, nq, nk, D, 77, 1000, orc)
    kc = (0.01 * rng.standard_normal((cap, nk * D))).astype(np.float32)
    kc[500] = 8.0
    q = np.ones(nq * D, np.float32)
    got = ring_call(hip, q, kc, vc, nq, nk, D, 0, 1024)
    for h in range(nq):
        assert np.array_equal(got[h], vc[500].reshape(nk, D)[h // 4])


def batched(hip, B, nq, nk, D, cap, starts, lens, rng, qs=None):
    import torch

    qs = qs or D
    q = rng.standard_normal((B, (nq - 1) * qs + D)).astype(np.float32)
    kc = rng.standard_normal((B, cap, nk * D)).astype(np.float32)
    vc = rng.standard_normal((B, cap, nk * D)).astype(np.float32)
    out = torch.full((B, nq * D), float("nan"), device="cuda")
    ws = torch.zeros(max(hip.gqa_workspace_size(B, nq, nk, D, cap), 1), dtype=torch.uint8, device="cuda")
    hip.gqa_attention(out, dev(q), dev(kc), dev(vc), dev(np.array(starts, np.int32)), dev(np.array(lens, np.int32)),
                      nq, nk, D, ws, q_head_stride=qs)
    return host(out).reshape(B, nq, D), q, kc, vc


def test_batched_decode_b64_full_shape(hip, orc, rng):
    """64 sequences at the Qwen3-8B decode shape (32 q heads, 8 kv heads,
    head_dim 128, capacity 2048) with different ring states."""
    B, nq, nk, D, cap = 64, 32, 8, 128, 2048
    starts = rng.integers(0, cap, B)
    lens = rng.integers(1, cap + 1, B)
    lens[:4] = [0, 1, cap, cap]
    starts[3] = 0
    got, q, kc, vc = batched(hip, B, nq, nk, D, cap, starts, lens, rng)
    for b in range(B):
        check(got[b], q[b], kc[b], vc[b], nq, nk, D, int(starts[b]), int(lens[b]), orc)


def test_whole_ring_threshold(hip, orc, rng):
    """Rings short enough for one workgroup (128 rows at this shape: 32-row
    chunks) are done by chunk 0 alone, longer ones split and merged; lengths
    on both sides of the threshold in one launch, some wrapping."""
    B, nq, nk, D, cap = 6, 16, 8, 128, 2048
    lens = [0, 1, 127, 128, 129, 2048]
    starts = [5, 2047, 1990, 0, 1950, 700]
    got, q, kc, vc = batched(hip, B, nq, nk, D, cap, starts, lens, rng)
    for b in range(B):
        check(got[b], q[b], kc[b], vc[b], nq, nk, D, starts[b], lens[b], orc)


@pytest.mark.parametrize("B,nq,nk,D,cap", [
    (64, 8, 8, 128, 1024),     # one q head per kv head, 512 pairs: whole-ring workgroups
    (63, 16, 8, 128, 1024),    # 504 pairs: split launch, the threshold's other side
    (128, 8, 4, 64, 300),      # head_dim 64, groups of 2
    (128, 16, 4, 256, 200),    # head_dim 256, groups of 4
    (64, 64, 8, 128, 256),     # groups of 8: above the whole-ring LDS budget, split launch
])
def test_whole_ring_launches(hip, orc, rng, B, nq, nk, D, cap):
    """At two or more (sequence, kv head) pairs per CU and rings of at most
    2048 rows, one workgroup per pair attends over its whole ring: ring
    states empty, single, full, wrapped and random, against the oracle."""
    starts = rng.integers(-cap, 2 * cap, B)
    lens = rng.integers(0, cap + 1, B)
    lens[:5] = [0, 1, cap, cap, cap - 1]
    starts[2] = 0
    got, q, kc, vc = batched(hip, B, nq, nk, D, cap, starts, lens, rng)
    for b in list(range(8)) + list(range(B - 8, B)):
        st = int(starts[b]) % cap
        check(got[b], q[b], kc[b], vc[b], nq, nk, D, st, int(lens[b]), orc)


@pytest.mark.parametrize("B,cap,lens", [(6, 2048, [0, 1, 127, 128, 129, 2048]), (3, 100, [1, 50, 100]),
                                       (3, 32, [1, 20, 32]), (64, 256, [0, 1, 256, 255] + [77] * 60)])
def test_fp16_output_is_fp32_output_rounded(hip, orc, rng, B, cap, lens):
    """The fp16-output attention writes the fp32 attention's values rounded
    to nearest even, bit for bit: whole rings written by chunk 0, split rings
    through the merge, a single-chunk launch, and one workgroup per ring at
    64 sequences."""
    import torch

    nq, nk, D = 16, 8, 128
    starts = [int(x) for x in rng.integers(0, cap, B)]
    q = dev(rng.standard_normal((B, nq * D)).astype(np.float32))
    kc = dev(rng.standard_normal((B, cap, nk * D)).astype(np.float32))
    vc = dev(rng.standard_normal((B, cap, nk * D)).astype(np.float32))
    ws = torch.zeros(max(hip.gqa_workspace_size(B, nq, nk, D, cap), 1), dtype=torch.uint8, device="cuda")
    st, ln = dev(np.array(starts, np.int32)), dev(np.array(lens, np.int32))
    o32 = torch.empty(B, nq * D, device="cuda")
    hip.gqa_attention(o32, q, kc, vc, st, ln, nq, nk, D, ws)
    o16 = torch.empty(B, nq * D, dtype=torch.int16, device="cuda")
    hip.gqa_attention(o16, q, kc, vc, st, ln, nq, nk, D, ws)
    assert_bitexact(host(o16), orc.f32_to_f16_rne(host(o32)).reshape(B, nq * D), "fp16 attention output")


@pytest.mark.parametrize("B,nq,nk,D,cap", [(3, 16, 8, 128, 4096), (600, 16, 8, 128, 64), (5, 8, 4, 64, 333)])
def test_batched_other_shapes(hip, orc, rng, B, nq, nk, D, cap):
    starts = rng.integers(0, cap, B)
    lens = rng.integers(0, cap + 1, B)
    got, q, kc, vc = batched(hip, B, nq, nk, D, cap, starts, lens, rng)
    for b in range(min(B, 40)):
        check(got[b], q[b], kc[b], vc[b], nq, nk, D, int(starts[b]), int(lens[b]), orc)


@pytest.mark.parametrize("B,cap,bound", [(1, 2048, 30), (1, 2048, 700), (64, 2048, 33), (3, 4096, 4096)])
def test_bounded_launch(hip, orc, rng, B, cap, bound):
    """Every ring no longer than the bound: the bounded launch (fewer chunks;
    no partials to merge when one chunk suffices) matches the oracle like the
    full one does."""
    import torch

    nq, nk, D = 16, 8, 128
    starts = rng.integers(0, cap, B).astype(np.int32)
    lens = rng.integers(0, bound + 1, B).astype(np.int32)
    lens[0] = bound
    q = rng.standard_normal((B, nq * D)).astype(np.float32)
    kc = rng.standard_normal((B, cap, nk * D)).astype(np.float32)
    vc = rng.standard_normal((B, cap, nk * D)).astype(np.float32)
    ws = torch.zeros(max(hip.gqa_workspace_size(B, nq, nk, D, cap), 16), dtype=torch.uint8, device="cuda")
    out = torch.empty(B, nq * D, device="cuda")
    hip.gqa_attention_bounded(out, dev(q), dev(kc), dev(vc), dev(starts), dev(lens), nq, nk, D, bound, ws)
    got = host(out).reshape(B, nq, D)
    for b in range(min(B, 8)):
        check(got[b], q[b], kc[b], vc[b], nq, nk, D, int(starts[b]), int(lens[b]), orc)


def test_ring_append_matches_oracle(hip, orc, rng):
    import torch

    B, nk, D, cap = 6, 8, 128, 16
    row = nk * D
    kc = rng.standard_normal((B, cap, row)).astype(np.float32)
    vc = rng.standard_normal((B, cap, row)).astype(np.float32)
    st = np.array([[0, 0], [3, 5], [15, 2], [0, 16], [9, 16], [7, 15]], np.int32)
    dk, dv = dev(kc), dev(vc)
    ds, dl = dev(st[:, 0].copy()), dev(st[:, 1].copy())
    for step in range(20):                                     # wraps every ring
        k = rng.standard_normal((B, row)).astype(np.float32)
        v = rng.standard_normal((B, row)).astype(np.float32)
        hip.kv_ring_append(dk, dv, ds, dl, dev(k), dev(v))
        for b in range(B):
            orc.kv_ring_append(kc[b], vc[b], k[b], v[b], st[b])
    assert np.array_equal(host(ds), st[:, 0]) and np.array_equal(host(dl), st[:, 1])
    assert_bitexact(host(dk), kc, "k cache")
    assert_bitexact(host(dv), vc, "v cache")


def test_append_then_attend_decode_loop(hip, orc, rng):
    """The decode loop of qwen3.cpp:475-492 for 2 sequences past the ring's
    capacity: append the token's k/v, then attend over the ring."""
    import torch

    B, nq, nk, D, cap = 2, 16, 8, 128, 24
    row = nk * D
    dk = torch.zeros(B, cap, row, device="cuda")
    dv = torch.zeros(B, cap, row, device="cuda")
    ds = torch.zeros(B, dtype=torch.int32, device="cuda")
    dl = torch.zeros(B, dtype=torch.int32, device="cuda")
    kc = np.zeros((B, cap, row), np.float32)
    vc = np.zeros((B, cap, row), np.float32)
    st = np.zeros((B, 2), np.int32)
    out = torch.empty(B, nq * D, device="cuda")
    ws = torch.zeros(max(hip.gqa_workspace_size(B, nq, nk, D, cap), 1), dtype=torch.uint8, device="cuda")
    for step in range(30):
        k = rng.standard_normal((B, row)).astype(np.float32)
        v = rng.standard_normal((B, row)).astype(np.float32)
        q = rng.standard_normal((B, nq * D)).astype(np.float32)
        hip.kv_ring_append(dk, dv, ds, dl, dev(k), dev(v))
        hip.gqa_attention(out, dev(q), dk, dv, ds, dl, nq, nk, D, ws)
        got = host(out).reshape(B, nq, D)
        for b in range(B):
            orc.kv_ring_append(kc[b], vc[b], k[b], v[b], st[b])
            check(got[b], q[b], kc[b], vc[b], nq, nk, D, int(st[b, 0]), int(st[b, 1]), orc)


def _ctr_region(ws_bytes):
    """The attention workspace's counter region: its last 64th, from a
    256-byte boundary (fixed by the workspace's size alone)."""
    return (ws_bytes - ws_bytes // 64) & ~255


def test_workspace_reuse_across_shapes(hip, orc, rng):
    """One workspace, sized for 64 sequences, serves a sequence of calls
    whose batch, chunking and ring lengths change (64, 1, 3 sequences; the
    ring form at a long, a short and again a long cache_len; a bounded call;
    64 again): every call against the oracle, and the counters are all back
    at zero at the end."""
    import torch

    nq, nk, D, cap = 32, 8, 128, 2048
    n = hip.gqa_workspace_size(64, nq, nk, D, cap)
    ws = torch.zeros(n, dtype=torch.uint8, device="cuda")

    def batched_call(B, lens):
        starts = rng.integers(0, cap, B).astype(np.int32)
        lens = np.asarray(lens, np.int32)
        q = rng.standard_normal((B, nq * D)).astype(np.float32)
        kc = rng.standard_normal((B, cap, nk * D)).astype(np.float32)
        vc = rng.standard_normal((B, cap, nk * D)).astype(np.float32)
        out = torch.full((B, nq * D), float("nan"), device="cuda")
        hip.gqa_attention(out, dev(q), dev(kc), dev(vc), dev(starts), dev(lens), nq, nk, D, ws)
        got = host(out).reshape(B, nq, D)
        for b in list(range(min(B, 4))) + [B - 1]:
            check(got[b], q[b], kc[b], vc[b], nq, nk, D, int(starts[b]), int(lens[b]), orc)

    def ring_call_ws(length):
        q = rng.standard_normal(nq * D).astype(np.float32)
        kc = rng.standard_normal((cap, nk * D)).astype(np.float32)
        vc = rng.standard_normal((cap, nk * D)).astype(np.float32)
        out = torch.full((nq, D), float("nan"), device="cuda")
        hip.gqa_attention_ring(out, dev(q), dev(kc), dev(vc), nq, nk, D, 7, length, ws)
        check(host(out), q, kc, vc, nq, nk, D, 7, length, orc)

    batched_call(64, rng.integers(129, cap + 1, 64))
    batched_call(1, [cap])
    batched_call(3, [1500, 200, cap])
    ring_call_ws(cap)
    ring_call_ws(300)
    ring_call_ws(cap)
    batched_call(64, rng.integers(129, cap + 1, 64))
    batched_call(2, [999, 130])
    torch.cuda.synchronize()
    ctr = host(ws)[_ctr_region(n):]
    assert not ctr.any(), "counters left non-zero"


def test_bounded_launch_ring_past_bound(hip, orc, rng):
    """A bounded launch given a ring longer than its bound attends over the
    launched chunks' positions only: one sequence, 8 kv heads and capacity
    2048 give 64-position chunks, so a bound of 200 launches 4 chunks and a
    700-row ring is attended over its first 256 positions.  The counters are
    left at zero: a full call on the same workspace afterwards is right."""
    import torch

    nq, nk, D, cap = 16, 8, 128, 2048
    n = hip.gqa_workspace_size(1, nq, nk, D, cap)
    ws = torch.zeros(n, dtype=torch.uint8, device="cuda")
    q = rng.standard_normal(nq * D).astype(np.float32)
    kc = rng.standard_normal((cap, nk * D)).astype(np.float32)
    vc = rng.standard_normal((cap, nk * D)).astype(np.float32)
    out = torch.full((1, nq * D), float("nan"), device="cuda")
    start = 1900
    hip.gqa_attention_bounded(out, dev(q[None]), dev(kc[None]), dev(vc[None]), dev(np.array([start], np.int32)),
                              dev(np.array([700], np.int32)), nq, nk, D, 200, ws)
    check(host(out).reshape(nq, D), q, kc, vc, nq, nk, D, start, 256, orc)
    for length in (700, 2048):
        hip.gqa_attention(out, dev(q[None]), dev(kc[None]), dev(vc[None]), dev(np.array([start], np.int32)),
                          dev(np.array([length], np.int32)), nq, nk, D, ws)
        check(host(out).reshape(nq, D), q, kc, vc, nq, nk, D, start, length, orc)
    torch.cuda.synchronize()
    assert not host(ws)[_ctr_region(n):].any(), "counters left non-zero"


def test_workspace_size_covers_smaller_batches(hip):
    """The size for a batch serves every smaller batch: the chunk grows with
    the batch, so a smaller batch can need more partials (three sequences at
    capacity 32768 need more than four)."""
    import torch

    nq, nk, D, cap = 32, 8, 128, 32768
    n4 = hip.gqa_workspace_size(4, nq, nk, D, cap)
    assert n4 >= hip.gqa_workspace_size(3, nq, nk, D, cap)
    ws = torch.zeros(n4, dtype=torch.uint8, device="cuda")
    q = torch.zeros(3, nq * D, device="cuda")
    out = torch.empty(3, nq * D, device="cuda")
    z = torch.zeros(3, dtype=torch.int32, device="cuda")    # empty rings: only the workspace check matters
    caches = torch.zeros(3, cap, nk * D, device="cuda")
    hip.gqa_attention(out, q, caches, caches, z, z, nq, nk, D, ws)
    assert not host(out).any()
