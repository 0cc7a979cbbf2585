"""Softmax (core/cpu_ops.cpp:83-99) and batched sample_token
(core/sampling.cpp:10-66) on the GPU.  Probabilities must be within 1e-5
relative (they are in fact bit-identical by construction, which is
asserted too) and token ids bit-exact given the same uniform draws."""
import ctypes
import ctypes.util
import json
import os

import numpy as np
import pytest

from helpers import REL_TOL, assert_bitexact, dev, host, max_rel_err

pytestmark = pytest.mark.gpu
GOLDEN = os.path.join(os.path.dirname(__file__), "golden")
V = 151936


def drand48_stream(seed, n):
    """r = (float)drand48() after srand48(seed): the reference's draws (main.cpp:196, sampling.cpp:58)."""
    libc = ctypes.CDLL(ctypes.util.find_library("c"))
    libc.drand48.restype = ctypes.c_double
    libc.srand48(ctypes.c_long(seed))
    return np.array([libc.drand48() for _ in range(n)], np.float64).astype(np.float32)


def run_sample(hip, logits, hist=None, hist_len=None, r=None, want_probs=True, **params):
    import torch

    rows, vocab = logits.shape
    p = hip.SamplingParams(**params)
    ids = torch.empty(rows, dtype=torch.int32, device="cuda")
    # the probability buffer is required when sampling (it is the draw's input)
    probs = torch.empty(rows, vocab, device="cuda") if (want_probs or p.temperature > 0) else None
    ws = torch.empty(hip.sample_workspace_size(rows, vocab), dtype=torch.uint8, device="cuda")
    hip.sample(ids, probs, dev(logits), dev(hist) if hist is not None else None,
               dev(hist_len) if hist_len is not None else None, p, dev(r) if r is not None else None, ws)
    return host(ids), (host(probs) if want_probs else None)


def oracle_rows(orc, logits, hist=None, hist_len=None, r=None, **params):
    ids, probs = [], []
    for i in range(logits.shape[0]):
        rec = None
        if hist is not None:
            n = hist.shape[1] if hist_len is None else int(hist_len[i])
            rec = hist[i, :n]
        tok, p = orc.sample_token(logits[i], recent=rec, r=float(r[i]) if r is not None else 0.0,
                                  want_probs=True, **params)
        ids.append(tok)
        probs.append(p)
    return np.array(ids), np.stack(probs)


@pytest.mark.parametrize("rows,n", [(1, 5), (3, V), (2, 1000), (4, 4096), (1, 4097), (2, 1)])
def test_softmax(hip, orc, rng, rows, n):
    import torch

    x = (rng.normal(0, 3, (rows, n)) / 0.6).astype(np.float32)
    t = dev(x)
    ws = torch.empty(hip.softmax_workspace_size(rows, n), dtype=torch.uint8, device="cuda")
    hip.softmax(t, ws)
    ref = np.stack([orc.softmax(row) for row in x])
    got = host(t)
    assert max_rel_err(got, ref) <= REL_TOL
    assert_bitexact(got, ref, "softmax")


def test_softmax_wide_range(hip, orc, rng):
    """x - max across [-160, 0]: exps that are subnormal, that round to zero,
    and the clamp's ends (-104 and its neighbours), bit-identical to the
    oracle, whose exp takes x < -104 and x > 89 as special cases."""
    import torch

    n = 8192
    x = rng.uniform(-160.0, 0.0, (3, n)).astype(np.float32)
    x[:, 0] = 0.0
    edges = np.array([-104.0, np.nextafter(np.float32(-104.0), np.float32(0.0)),
                      np.nextafter(np.float32(-104.0), np.float32(-200.0)), -103.97, -103.28, -87.3365,
                      -87.3366, -88.0, -100.0, -149.0, -1e30], np.float32)
    x[0, 1:1 + len(edges)] = edges
    x[2] += np.float32(30.0)  # max 30: shifted inputs give the same differences
    t = dev(x)
    ws = torch.empty(hip.softmax_workspace_size(3, n), dtype=torch.uint8, device="cuda")
    hip.softmax(t, ws)
    ref = np.stack([orc.softmax(row) for row in x])
    got = host(t)
    assert (got[0, 1:4] >= 0).all() and got[0, 3] == 0.0  # below -104: exactly zero
    assert ((got > 0) & (got < np.finfo(np.float32).tiny)).any()  # subnormal results occur
    assert_bitexact(got, ref, "softmax wide range")


@pytest.mark.parametrize("freq", [0.1, 0.0])
def test_sampler_full_config(hip, orc, rng, freq):
    """Logits [64, 151936] ~N(0,3), history [64, 256] ~U[0,V), rep 1.2, T 0.6."""
    logits = rng.normal(0, 3, (64, V)).astype(np.float32)
    hist = rng.integers(0, V, (64, 256)).astype(np.int32)
    r = drand48_stream(1234, 64)
    ids, probs = run_sample(hip, logits, hist, r=r, temperature=0.6, repetition_penalty=1.2,
                            repetition_context_size=256, frequency_penalty=freq)
    rids, rprobs = oracle_rows(orc, logits, hist, r=r, temperature=0.6, repetition_penalty=1.2,
                               repetition_context_size=256, frequency_penalty=freq)
    assert max_rel_err(probs, rprobs) <= REL_TOL
    assert_bitexact(probs, rprobs, "probabilities")
    assert np.array_equal(ids, rids)


@pytest.mark.parametrize("rows", [8, 1])
def test_sampler_nan_and_inf_logits_full_vocab(hip, orc, rng, rows):
    """Rows of 151936 logits, where the exact per-lane sums run in fp64 (chunks
    of 3072 at 8 rows, of 1024 at one row), with a NaN, a +inf and -inf
    logits: ids equal the oracle's; probabilities are NaN exactly where the
    oracle's are and bit-identical elsewhere."""
    logits = rng.normal(0, 3, (rows, V)).astype(np.float32)
    logits[0, 5] = np.nan
    if rows > 1:
        logits[1, V - 1] = np.nan      # in the last, partial chunk
        logits[2, 1000] = np.inf
        logits[3, ::7] = -np.inf
        logits[4, 77777] = np.nan
    hist = rng.integers(0, V, (rows, 256)).astype(np.int32)
    r = drand48_stream(99, rows)
    params = dict(temperature=0.6, repetition_penalty=1.2, repetition_context_size=256, frequency_penalty=0.1)
    ids, probs = run_sample(hip, logits, hist, r=r, **params)
    rids, rprobs = oracle_rows(orc, logits, hist, r=r, **params)
    assert np.array_equal(ids, rids)
    gn, rn = np.isnan(probs), np.isnan(rprobs)
    assert np.array_equal(gn, rn)
    assert rn[0].all() and ids[0] == V - 1
    assert_bitexact(np.where(gn, 0.0, probs).astype(np.float32), np.where(rn, 0.0, rprobs).astype(np.float32),
                    "probabilities")


def test_sampler_draws_on_cdf_boundaries(hip, orc, rng):
    """r set to exact running-sum values and their neighbours: any
    deviation from the sequential fp32 walk changes the id."""
    rows = 64
    logits = (rng.normal(0, 3, (rows, 20000))).astype(np.float32)
    _, base = oracle_rows(orc, logits, r=np.zeros(rows, np.float32), temperature=0.6, frequency_penalty=0.0)
    r = np.empty(rows, np.float32)
    for i in range(rows):
        cum = np.add.accumulate(base[i], dtype=np.float32)
        k = int(rng.integers(0, cum.size))
        r[i] = [cum[k], np.nextafter(cum[k], np.float32(2)), np.nextafter(cum[k], np.float32(-1)),
                np.nextafter(cum[-1], np.float32(2)), cum[-1], np.float32(0)][i % 6]
    ids, _ = run_sample(hip, logits, r=r, temperature=0.6, frequency_penalty=0.0, want_probs=False)
    rids, _ = oracle_rows(orc, logits, r=r, temperature=0.6, frequency_penalty=0.0)
    assert np.array_equal(ids, rids)


def test_sampler_many_binades_and_ties(hip, orc, rng):
    """Rows whose probabilities make the running sum cross many binades and
    hit exact half-ulp ties: logits on a coarse grid give repeated values."""
    rows, n = 32, 6000
    logits = (np.round(rng.normal(0, 2, (rows, n)) * 2) / 2).astype(np.float32)
    logits[::4, :3] = 30.0          # dominant leading tokens: absorption right away
    logits[1::4, -3:] = 30.0        # dominant trailing tokens
    r = rng.uniform(0, 1, rows).astype(np.float32)
    ids, probs = run_sample(hip, logits, r=r, temperature=1.0, frequency_penalty=0.0)
    rids, rprobs = oracle_rows(orc, logits, r=r, temperature=1.0, frequency_penalty=0.0)
    assert_bitexact(probs, rprobs, "probabilities")
    assert np.array_equal(ids, rids)


def test_sampler_history_lengths_and_window(hip, orc, rng):
    rows, n = 8, 3000
    logits = rng.normal(0, 3, (rows, n)).astype(np.float32)
    hist = rng.integers(-5, n + 5, (rows, 300)).astype(np.int32)   # includes out-of-range ids
    hist[:, :150] = hist[:, :1]                                    # heavy duplicates
    hl = np.array([0, 1, 10, 255, 256, 257, 299, 300], np.int32)
    r = rng.uniform(0, 1, rows).astype(np.float32)
    for ctx in (256, 7):
        ids, probs = run_sample(hip, logits, hist, hl, r, temperature=0.8, repetition_penalty=1.3,
                                repetition_context_size=ctx, frequency_penalty=0.25)
        rids, rprobs = oracle_rows(orc, logits, hist, hl, r, temperature=0.8, repetition_penalty=1.3,
                                   repetition_context_size=ctx, frequency_penalty=0.25)
        assert_bitexact(probs, rprobs, f"ctx {ctx}")
        assert np.array_equal(ids, rids)


def test_sampler_argmax_path(hip, orc, rng):
    rows, n = 6, 9000
    logits = np.round(rng.normal(0, 1, (rows, n)) * 4).astype(np.float32)  # many ties
    logits[2, 0] = np.nan           # NaN at index 0 is never replaced
    logits[3, 5] = np.nan           # NaN elsewhere is skipped
    logits[4, :] = -np.inf          # all -inf: first index
    hist = rng.integers(0, n, (rows, 64)).astype(np.int32)
    ids, _ = run_sample(hip, logits, hist, temperature=0.0, want_probs=False)
    rids, _ = oracle_rows(orc, logits, hist, temperature=0.0)
    assert np.array_equal(ids, rids)


def test_sampler_nan_logit_gives_last_id(hip, orc, rng):
    logits = rng.normal(0, 1, (2, 777)).astype(np.float32)
    logits[0, 100] = np.nan
    r = np.array([0.5, 0.5], np.float32)
    ids, probs = run_sample(hip, logits, r=r)
    rids, _ = oracle_rows(orc, logits, r=r)
    assert np.array_equal(ids, rids) and ids[0] == 776
    assert np.all(np.isnan(probs[0]))


def _kats():
    with open(os.path.join(GOLDEN, "sampler_kat.json")) as f:
        return json.load(f)["cases"]


@pytest.mark.parametrize("case", _kats(), ids=lambda c: c["name"])
def test_sampler_known_answers(hip, case):
    if case.get("generator") == "dominant_first":
        logits = np.zeros(case["n_small"] + 1, np.float32)
        logits[0] = case["big"]
    else:
        logits = np.array(case["logits"], np.float32)
    rec = np.array(case.get("recent", []), np.int32)
    ids, _ = run_sample(hip, logits[None], rec[None] if rec.size else None, r=np.array([case.get("r", 0.0)], np.float32),
                        want_probs=False, temperature=case.get("temperature", 0.6),
                        repetition_penalty=case.get("repetition_penalty", 1.2),
                        repetition_context_size=case.get("repetition_context_size", 256),
                        frequency_penalty=case.get("frequency_penalty", 0.1))
    assert int(ids[0]) == case["expect"], case["why"]


def test_sampler_leaves_logits_unchanged(hip, rng):
    import torch

    logits = rng.normal(0, 3, (4, 5000)).astype(np.float32)
    lt = dev(logits)
    p = hip.SamplingParams()
    ids = torch.empty(4, dtype=torch.int32, device="cuda")
    probs = torch.empty(4, 5000, device="cuda")
    ws = torch.empty(hip.sample_workspace_size(4, 5000), dtype=torch.uint8, device="cuda")
    hip.sample(ids, probs, lt, dev(rng.integers(0, 5000, (4, 256)).astype(np.int32)), None, p,
               dev(np.full(4, 0.5, np.float32)), ws)
    assert np.array_equal(host(lt), logits)


@pytest.mark.parametrize("rows", [8, 32])
def test_sampler_row_alignments_agree(hip, orc, rng, rows):
    """Logits rows and probability rows each 16-byte aligned or starting one
    float off (the element-wise loads, stores, or both; at 32 rows aligned
    inputs take the one launch, the others the three launches): ids and
    probabilities bit-identical across all four, and the ids equal to the
    oracle's."""
    import torch

    logits = rng.normal(0, 3, (rows, V)).astype(np.float32)
    hist = rng.integers(0, V, (rows, 256)).astype(np.int32)
    r = drand48_stream(31, rows)
    p = hip.SamplingParams(temperature=0.6, repetition_penalty=1.2, repetition_context_size=256,
                           frequency_penalty=0.1)
    ws = torch.empty(hip.sample_workspace_size(rows, V), dtype=torch.uint8, device="cuda")
    out = {}
    for off_in in (0, 1):
        lbuf = torch.zeros(rows * V + 4, device="cuda")
        lg = lbuf[off_in:off_in + rows * V].view(rows, V)
        lg.copy_(dev(logits))
        for off_out in (0, 1):
            pbuf = torch.full((rows * V + 4,), float("nan"), device="cuda")
            pr = pbuf[off_out:off_out + rows * V].view(rows, V)
            ids = torch.full((rows,), -7, dtype=torch.int32, device="cuda")
            hip.sample(ids, pr, lg, dev(hist), None, p, dev(r), ws)
            out[(off_in, off_out)] = (host(ids), host(pr))
    base_ids, base_probs = out[(0, 0)]
    for key, (ids, probs) in out.items():
        assert np.array_equal(ids, base_ids), key
        assert_bitexact(probs, base_probs, f"offsets {key}")
    rids, _ = oracle_rows(orc, logits, hist, r=r, temperature=0.6, repetition_penalty=1.2,
                          repetition_context_size=256, frequency_penalty=0.1)
    assert np.array_equal(base_ids, rids)
