"""The op chain captured into a HIP graph (as bench.py runs it) gives, on
every replay, exactly what the same launches give eagerly.  Replays are
separated by unrelated eager work and synchronisations."""
import numpy as np
import pytest

from helpers import dev, gamma_f16, host

pytestmark = pytest.mark.gpu
D, THETA, EPS = 128, 1e6, 1e-6


def _state(rng_seed, T, H, nq, nk, I, V):
    r = np.random.default_rng(rng_seed)
    st = dict(x=r.standard_normal((T, H), dtype=np.float32), attn=r.standard_normal((T, H), dtype=np.float32),
              mlp=r.standard_normal((T, H), dtype=np.float32), q=r.standard_normal((T, nq * D), dtype=np.float32),
              k=r.standard_normal((T, nk * D), dtype=np.float32), g=r.standard_normal((T, I), dtype=np.float32),
              u=r.standard_normal((T, I), dtype=np.float32), table=gamma_f16(r, (V, H)),
              ids=r.integers(0, V, T).astype(np.int32), pos=r.integers(0, 32768, T).astype(np.int32),
              w_in=gamma_f16(r, H), w_post=gamma_f16(r, H), wq=gamma_f16(r, D), wk=gamma_f16(r, D))
    return st


def _to_dev(st):
    import torch

    d = {}
    for k, v in st.items():
        t = dev(v)
        d[k] = t.view(torch.float16) if v.dtype == np.uint16 else t
    d["xn"] = torch.empty_like(d["x"])
    d["h"] = torch.empty_like(d["g"])
    return d


def _layer(hip, d, cos, sin, nq, nk):
    hip.embed_gather(d["x"], d["table"], d["ids"])
    hip.rmsnorm(d["xn"], d["x"], d["w_in"], EPS)
    hip.qknorm_rope(d["q"], d["k"], d["wq"], d["wk"], d["pos"], cos, sin, THETA, EPS, nq=nq, nk=nk)
    hip.add_rmsnorm(d["x"], d["attn"], d["xn"], d["w_post"], EPS)
    hip.silu_mul(d["h"], d["g"], d["u"])
    hip.residual_add(d["x"], d["mlp"])


def test_graph_replays_match_eager(hip):
    import torch

    T, H, nq, nk, I, V = 64, 2560, 32, 8, 9728, 4096
    st = _state(5, T, H, nq, nk, I, V)
    eager, graphed = _to_dev(st), _to_dev(st)
    cos, sin = torch.empty(16384, 64, device="cuda"), torch.empty(16384, 64, device="cuda")
    hip.rope_table(cos, sin, THETA)
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        _layer(hip, graphed, cos, sin, nq, nk)
    torch.cuda.synchronize()
    # capture does not execute: graphed state is still the initial state
    assert np.array_equal(host(graphed["q"]), st["q"])
    scratch = torch.randn(1 << 20, device="cuda")
    for rep in range(4):
        _layer(hip, eager, cos, sin, nq, nk)
        g.replay()
        scratch.mul_(1.0001)                         # unrelated eager work between replays
        hip.residual_add(scratch, scratch)
        torch.cuda.synchronize()
        for name in ("x", "xn", "q", "k", "h"):
            assert np.array_equal(host(eager[name]).view(np.uint32), host(graphed[name]).view(np.uint32)), \
                f"replay {rep}: {name} differs from eager"


@pytest.mark.parametrize("rows,V", [(3, 20000), (16, 20000), (64, 151936)])
def test_sampler_graph_replays_match_eager(hip, rng, rows, V):
    """From 12 rows the sampler is one launch for stages 1-3 (chunks of 4
    k-slices at 16 rows here, 8 at 64) whose row barriers take their token
    from the workspace's epoch, which the walk advances on the device; at 3
    rows it is three launches and the epoch stays.  Every replay of the
    captured call (new logits and draws each time) matches the eager call."""
    import torch

    logits = dev(rng.normal(0, 3, (rows, V)).astype(np.float32))
    hist = dev(rng.integers(0, V, (rows, 256)).astype(np.int32))
    r = dev(rng.uniform(0, 1, rows).astype(np.float32))
    p = hip.SamplingParams()
    ws_e = torch.empty(hip.sample_workspace_size(rows, V), dtype=torch.uint8, device="cuda")
    ws_g = torch.empty_like(ws_e)
    ids_e, ids_g = torch.empty(rows, dtype=torch.int32, device="cuda"), torch.empty(rows, dtype=torch.int32, device="cuda")
    pr_e, pr_g = torch.empty(rows, V, device="cuda"), torch.empty(rows, V, device="cuda")
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        hip.sample(ids_g, pr_g, logits, hist, None, p, r, ws_g)
    epoch = lambda ws: int(host(ws[:8]).view(np.uint64)[0])
    e0 = epoch(ws_g)
    for rep in range(3):
        r.copy_(torch.rand(rows, device="cuda"))      # new draws each step, read by both
        logits.normal_(0.0, 3.0)                      # and new logits
        hip.sample(ids_e, pr_e, logits, hist, None, p, r, ws_e)
        g.replay()
        torch.cuda.synchronize()
        assert np.array_equal(host(ids_e), host(ids_g)), f"replay {rep}: ids"
        assert np.array_equal(host(pr_e).view(np.uint32), host(pr_g).view(np.uint32)), f"replay {rep}: probs"
        assert epoch(ws_g) == ((e0 + rep + 1) % (1 << 64) if rows >= 12 else e0), f"replay {rep}: epoch"
        assert host(ids_g).min() >= 0


@pytest.mark.parametrize("B,steps,V", [(1, 140, 300), (3, 30, 300), (20, 24, 300), (20, 8, 70000), (9, 8, 300)])
def test_decode_step_graph_replays_match_eager(hip, rng, tmp_path, B, steps, V):
    """The Qwen3 decode step captured once (positions advanced inside the
    graph, as bench.py runs it) gives on every replay the logits of the same
    step run eagerly on a twin model, bit for bit: one sequence (dot-kernel
    projections; its rings pass the 128-row whole-ring limit of the
    attention), three (MFMA), twenty (fp16-row projections, fp16
    attention output), twenty with a 70000-row LM head (the branch of
    Qwen3's 151936-row vocabulary), and nine with an intermediate size that
    is not a multiple of 32 (the per-op branch)."""
    import torch

    from helpers import save_qwen3, tiny_qwen3

    t, d = tiny_qwen3(rng, tied=False, V=V, I=336 if B == 9 else 384)
    path = tmp_path / "tiny.safetensors"
    save_qwen3(path, t)
    cfg = hip.Qwen3Config(d["H"], d["L"], d["nq"], d["nk"], d["D"], d["I"], d["V"], 1e6, 1e-6)
    eager = hip.Qwen3Model(path, cfg, max_batch=B, kv_capacity=256)
    graph = hip.Qwen3Model(path, cfg, max_batch=B, kv_capacity=256)
    ids = dev(rng.integers(0, d["V"], B).astype(np.int32))
    pos_e = dev(np.resize(np.array([0, 7, 20000], np.int32), B))
    pos_g = pos_e.clone()
    le = torch.empty(B, d["V"], device="cuda")
    lg = torch.empty(B, d["V"], device="cuda")
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        graph.forward(ids, pos_g, lg)
        pos_g.add_(1)
    for s in range(steps):
        eager.forward(ids, pos_e, le)
        pos_e.add_(1)
        g.replay()
        torch.cuda.synchronize()
        assert np.array_equal(host(le).view(np.uint32), host(lg).view(np.uint32)), f"step {s}"
    eager.close()
    graph.close()
