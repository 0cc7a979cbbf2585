"""The sampler's one-launch path (stages 1-3 in one kernel with per-row
barriers), which anelm_sample takes from 12 rows when the rows are 16-byte
aligned and the grid fits on the GPU at once (chunks of 4, 8 or 12 k-slices,
the smallest that fits: 4 up to 40 rows of 151936, 8 up to 64, 12 up to 74):
token ids bit-exact against the
oracle (core/sampling.cpp:10-66) and probabilities bit-identical, on the edge
cases the three-launch path is tested on, on workspaces that start with
arbitrary contents and are reused across shapes, and bit-identical to the
three-launch path itself (taken for the same rows when the probability rows
are not 16-byte aligned)."""
import numpy as np
import pytest

from helpers import assert_bitexact, dev, host
from test_gpu_sampling import V, drand48_stream, oracle_rows

pytestmark = pytest.mark.gpu

PARAMS = dict(temperature=0.6, repetition_penalty=1.2, repetition_context_size=256, frequency_penalty=0.1)


def _rows4(a):
    """[rows, vocab] float32 on the device in rows of a multiple of 4 floats
    (16-byte aligned rows, whatever the vocabulary)."""
    import torch

    rows, vocab = a.shape
    buf = torch.zeros(rows, (vocab + 3) // 4 * 4, device="cuda")
    buf[:, :vocab] = dev(np.ascontiguousarray(a))
    return buf[:, :vocab]


def _call(hip, logits, ws, hist=None, hist_len=None, r=None, ld_pad=0, **params):
    """anelm_sample with the given workspace on 16-byte aligned logits rows;
    probability rows aligned too, or with ld_pad = 1 one float longer
    (unaligned: the three launches)."""
    import torch

    rows, vocab = logits.shape
    p = hip.SamplingParams(**params)
    ids = torch.full((rows,), -7, dtype=torch.int32, device="cuda")
    pbuf = torch.full((rows, (vocab + 3) // 4 * 4 + ld_pad), float("nan"), device="cuda")
    probs = pbuf[:, :vocab]
    hip.sample(ids, probs, _rows4(logits), dev(hist) if hist is not None else None,
               dev(hist_len) if hist_len is not None else None, p, dev(r), ws)
    return host(ids), host(probs)


def _epoch(ws):
    """The workspace's first 8 bytes: one-launch calls made on it."""
    return int(host(ws[:8]).view(np.uint64)[0])


def _check(ids, probs, rids, rprobs, what):
    assert np.array_equal(ids, rids), what
    gn, rn = np.isnan(probs), np.isnan(rprobs)
    assert np.array_equal(gn, rn), what
    assert_bitexact(np.where(gn, 0.0, probs).astype(np.float32), np.where(rn, 0.0, rprobs).astype(np.float32), what)


def test_fused_path_taken_from_12_rows(hip, orc, rng):
    """The epoch in the workspace's first word counts one-launch calls: it
    advances once per call at 72, 48, 16 and 12 rows (chunks of 12, 8, 4 and
    4 k-slices) and stays put at 11 rows (three launches), and the ids and
    probabilities match the oracle each time."""
    import torch

    ws = torch.zeros(hip.sample_workspace_size(72, V), dtype=torch.uint8, device="cuda")
    expect = 0
    for rows, fused in ((72, True), (48, True), (16, True), (12, True), (11, False), (64, True)):
        logits = rng.normal(0, 3, (rows, V)).astype(np.float32)
        hist = rng.integers(0, V, (rows, 256)).astype(np.int32)
        r = rng.uniform(0, 1, rows).astype(np.float32)
        ids, probs = _call(hip, logits, ws, hist, r=r, **PARAMS)
        expect += 1 if fused else 0
        assert _epoch(ws) == expect, (rows, _epoch(ws))
        rids, rprobs = oracle_rows(orc, logits, hist, r=r, **PARAMS)
        _check(ids, probs, rids, rprobs, f"{rows} rows")


@pytest.mark.parametrize("rows", [16, 44, 64, 72])
def test_fused_equals_three_launches(hip, rng, rows):
    """The same rows through both paths (unaligned probability rows take the
    three launches), at each one-launch chunk size (4, 8 and 12 k-slices at
    16, 64 and 72 rows; 44 rows fit chunks of 4 only past their 85% limit, so
    take 8): ids and probabilities bit-identical."""
    import torch

    logits = rng.normal(0, 3, (rows, V)).astype(np.float32)
    hist = rng.integers(0, V, (rows, 256)).astype(np.int32)
    r = drand48_stream(7, rows)
    ws = torch.empty(hip.sample_workspace_size(rows, V), dtype=torch.uint8, device="cuda")
    ws.fill_(0xFF)
    a_ids, a_probs = _call(hip, logits, ws, hist, r=r, **PARAMS)
    assert _epoch(ws) == 0          # 0xFF..FF + 1 wraps: one one-launch call made
    b_ids, b_probs = _call(hip, logits, ws, hist, r=r, ld_pad=1, **PARAMS)
    assert _epoch(ws) == 0          # the three launches leave it
    assert np.array_equal(a_ids, b_ids)
    assert_bitexact(a_probs, b_probs, "one launch against three")


def test_fused_nan_inf_and_history_lengths(hip, orc, rng):
    """48 rows of 151936: NaN, +inf and -inf logits (one in the last, partial
    chunk), device history lengths from 0 to the whole history, out-of-range
    and repeated ids, against the oracle."""
    rows = 48
    logits = rng.normal(0, 3, (rows, V)).astype(np.float32)
    logits[0, 5] = np.nan
    logits[1, V - 1] = np.nan
    logits[2, 1000] = np.inf
    logits[3, ::7] = -np.inf
    logits[4, 77777] = np.nan
    logits[5, 12287:12290] = np.inf       # across a chunk boundary
    hist = rng.integers(-5, V + 5, (rows, 300)).astype(np.int32)
    hist[6:9, :150] = hist[6:9, :1]       # heavy duplicates
    hl = rng.integers(0, 301, rows).astype(np.int32)
    hl[:4] = [0, 1, 256, 300]
    r = drand48_stream(99, rows)
    for ctx in (256, 7):
        params = dict(PARAMS, repetition_context_size=ctx, frequency_penalty=0.25)
        ids, probs = _call(hip, logits, _ws(hip, rows, V), hist, hl, r, **params)
        rids, rprobs = oracle_rows(orc, logits, hist, hl, r, **params)
        _check(ids, probs, rids, rprobs, f"ctx {ctx}")
        assert ids[0] == V - 1


def _ws(hip, rows, vocab):
    import torch

    return torch.empty(hip.sample_workspace_size(rows, vocab), dtype=torch.uint8, device="cuda")


@pytest.mark.parametrize("vocab", [12289, 4099, 24576, 8])
def test_fused_vocab_shapes(hip, orc, rng, vocab):
    """Vocabularies of one chunk and a single element (12289), not a multiple
    of 4 (4099; the kernel's element-wise loads), exactly two chunks (24576)
    and tiny (8), at 48 rows, each through the one launch (the epoch
    advances)."""
    rows = 48
    logits = (rng.normal(0, 3, (rows, vocab)) / 0.6).astype(np.float32)
    hist = rng.integers(0, vocab, (rows, 64)).astype(np.int32)
    r = rng.uniform(0, 1, rows).astype(np.float32)
    r[0] = 0.0
    r[1] = np.float32(1.0 - 2.0 ** -24)
    ws = _ws(hip, rows, vocab)
    e0 = _epoch(ws)
    ids, probs = _call(hip, logits, ws, hist, r=r, **PARAMS)
    assert _epoch(ws) == (e0 + 1) % (1 << 64), f"vocab {vocab}: the one-launch path was not taken"
    rids, rprobs = oracle_rows(orc, logits, hist, r=r, **PARAMS)
    _check(ids, probs, rids, rprobs, f"vocab {vocab}")


def test_fused_workspace_reused_across_shapes(hip, orc, rng):
    """One workspace that starts as random bytes serves calls of 64, 48 and
    56 rows over three vocabularies, then 64 rows again: every call matches
    the oracle (flags left by a call of another shape never pass a barrier)."""
    import torch

    cap = max(hip.sample_workspace_size(64, V), hip.sample_workspace_size(56, 50000))
    ws = torch.from_numpy(rng.integers(0, 256, cap, dtype=np.uint8)).cuda()
    e0 = _epoch(ws)
    for k, (rows, vocab) in enumerate(((64, V), (48, 50000), (56, 9000), (64, V))):
        logits = rng.normal(0, 3, (rows, vocab)).astype(np.float32)
        hist = rng.integers(0, vocab, (rows, 256)).astype(np.int32)
        r = rng.uniform(0, 1, rows).astype(np.float32)
        ids, probs = _call(hip, logits, ws, hist, r=r, **PARAMS)
        rids, rprobs = oracle_rows(orc, logits, hist, r=r, **PARAMS)
        _check(ids, probs, rids, rprobs, f"call {k}: {rows} x {vocab}")
        assert _epoch(ws) == (e0 + k + 1) % (1 << 64)


def test_long_window_takes_three_launches(hip, orc, rng):
    """A window of more than 65535 ids (its counts would not fit 16 bits)
    makes anelm_sample take the three launches at 48 rows: the epoch stays
    put and the results match the oracle."""
    import torch

    rows, vocab, n = 48, 6000, 70000
    logits = rng.normal(0, 3, (rows, vocab)).astype(np.float32)
    hist = rng.integers(0, vocab, (rows, n)).astype(np.int32)
    hist[:, : n // 2] = hist[:, :1]            # one id counted 35000 times and more
    r = rng.uniform(0, 1, rows).astype(np.float32)
    params = dict(PARAMS, repetition_context_size=n)
    ws = torch.zeros(hip.sample_workspace_size(rows, vocab), dtype=torch.uint8, device="cuda")
    ids, probs = _call(hip, logits, ws, hist, r=r, **params)
    assert _epoch(ws) == 0
    rids, rprobs = oracle_rows(orc, logits, hist, r=r, **params)
    _check(ids, probs, rids, rprobs, "window of 70000")
    # the same rows with a window of 65535 take the one launch
    params = dict(PARAMS, repetition_context_size=65535)
    ids, probs = _call(hip, logits, ws, hist, r=r, **params)
    assert _epoch(ws) == 1
    rids, rprobs = oracle_rows(orc, logits, hist, r=r, **params)
    _check(ids, probs, rids, rprobs, "window of 65535")


def test_concurrent_calls_on_four_streams(hip, rng):
    """Four 64-row one-launch calls issued at once on four streams (together
    four times the workgroups the GPU holds at once, so their grids cannot be
    resident together): every call still returns what it returns alone,
    bit for bit, and no row comes back -1 (a row barrier that gave up)."""
    import torch

    rows, V, n = 64, 151936, 4
    p = hip.SamplingParams()
    logits = [dev(rng.normal(0, 3, (rows, V)).astype(np.float32)) for _ in range(n)]
    hist = [dev(rng.integers(0, V, (rows, 256)).astype(np.int32)) for _ in range(n)]
    r = [dev(rng.uniform(0, 1, rows).astype(np.float32)) for _ in range(n)]
    ws = [torch.empty(hip.sample_workspace_size(rows, V), dtype=torch.uint8, device="cuda") for _ in range(n)]
    ids = [torch.full((rows,), -7, dtype=torch.int32, device="cuda") for _ in range(n)]
    probs = [torch.empty(rows, V, device="cuda") for _ in range(n)]
    ref = []
    for i in range(n):   # each alone
        hip.sample(ids[i], probs[i], logits[i], hist[i], None, p, r[i], ws[i])
        torch.cuda.synchronize()
        ref.append((host(ids[i]), host(probs[i])))
    streams = [torch.cuda.Stream() for _ in range(n)]
    for rep in range(3):
        for i in range(n):
            ids[i].fill_(-7)
        torch.cuda.synchronize()
        for i in range(n):   # all at once
            with torch.cuda.stream(streams[i]):
                hip.sample(ids[i], probs[i], logits[i], hist[i], None, p, r[i], ws[i])
        torch.cuda.synchronize()
        for i in range(n):
            got = host(ids[i])
            assert got.min() >= 0, f"rep {rep}, call {i}: a row barrier gave up"
            assert np.array_equal(got, ref[i][0]), f"rep {rep}, call {i}: ids"
            assert np.array_equal(host(probs[i]).view(np.uint32), ref[i][1].view(np.uint32)), f"rep {rep}, call {i}"
