"""anelm_sample_noalloc (the sampler with its workspace in the library's
static per-GPU scratch, for callers that cannot allocate) against
anelm_sample with a caller workspace, through the C ABI: ids and
probabilities bit-identical, on two calls in a row (the second with fewer
rows and a smaller vocabulary, so the scratch holds the first call's
leftovers), on the argmax path, and past the scratch's size limit."""
import numpy as np
import pytest

from helpers import dev, host

pytestmark = pytest.mark.gpu


def _inputs(rng, rows, V):
    logits = dev(rng.normal(0, 3, (rows, V)).astype(np.float32))
    hist = dev(rng.integers(0, V, (rows, 256)).astype(np.int32))
    r = dev(rng.uniform(0, 1, rows).astype(np.float32))
    return logits, hist, r


def _both(hip, logits, hist, r, p):
    import torch

    rows, V = logits.shape
    out = {}
    for name in ("ws", "noalloc"):
        ids = torch.full((rows,), -7, dtype=torch.int32, device="cuda")
        probs = torch.full((rows, V), float("nan"), device="cuda")
        if name == "ws":
            ws = torch.empty(hip.sample_workspace_size(rows, V), dtype=torch.uint8, device="cuda")
            hip.sample(ids, probs, logits, hist, None, p, r, ws)
        else:
            hip.sample_noalloc(ids, probs, logits, hist, None, p, r)
        out[name] = (host(ids), host(probs))
    return out


def test_noalloc_matches_workspace_sampler_twice(hip, rng):
    p = hip.SamplingParams()
    for rows, V in ((64, 151936), (5, 50000)):       # the second call smaller than the first
        logits, hist, r = _inputs(rng, rows, V)
        o = _both(hip, logits, hist, r, p)
        assert np.array_equal(o["ws"][0], o["noalloc"][0]), f"ids differ at {rows}x{V}"
        assert np.array_equal(o["ws"][1].view(np.uint32), o["noalloc"][1].view(np.uint32)), f"probs at {rows}x{V}"
        assert np.all((o["noalloc"][0] >= 0) & (o["noalloc"][0] < V))


def test_noalloc_argmax_path(hip, rng):
    p = hip.SamplingParams(temperature=0.0)
    for rows, V in ((33, 151936), (2, 1000)):
        logits, hist, r = _inputs(rng, rows, V)
        o = _both(hip, logits, hist, r, p)
        assert np.array_equal(o["ws"][0], o["noalloc"][0])


def test_noalloc_rejects_sizes_past_the_scratch(hip, rng):
    import torch

    V = 151936
    assert hip.sample_workspace_size(181, V) <= 4 << 20 < hip.sample_workspace_size(182, V)
    logits = torch.zeros(187, V, device="cuda")
    ids = torch.full((187,), -7, dtype=torch.int32, device="cuda")
    probs = torch.empty(187, V, device="cuda")
    r = torch.full((187,), 0.5, device="cuda")
    with pytest.raises(hip.AnelmError, match="scratch"):
        hip.sample_noalloc(ids, probs, logits, None, None, hip.SamplingParams(), r)
    assert np.all(host(ids) == -7)                     # nothing was launched
