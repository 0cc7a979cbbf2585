"""Benchmark of the fused layer-op path on one MI355X.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--workload NAME]

A step is one pass of the op chain over all layers of the headline workload
(the Qwen3-8B-shaped prefill, T=8192, 36 layers):
  (1) RMSNorm  (2) q/k-norm + RoPE  (3) residual add + RMSNorm
  (4) SwiGLU   (5) residual add
(the ops of models/llm/qwen3.cpp:502-528) on synthetic device-resident
inputs, distinct per layer, with the residual stream and the outputs rotating
over four buffer sets.  The headline step runs op-major: each op over all 36
layers is one HIP graph, replayed `steps` times after `warmup`, and the step
time is the sum of the five; no launch then reads what the launch before it
wrote, so every byte counted comes from HBM, not from the 256 MB Infinity
Cache.  `value` is the chain's algorithmic HBM bytes per step divided by
that step time.  The layer-major chain (the model's order, one graph per
step), in which an op can read part of its input from the Infinity Cache,
is reported beside it as `layer_major_chain`.
The same JSON line also reports the other configurations (0.6B decode and
prefill, 4B batched decode, the sampling tail, the bf16->fp16 convert of the
8.19 B-parameter set) and the CPU oracle timed on this host.
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(ROOT, "ane-lm_amd"))

HBM_PEAK_GBPS = 8000.0
METRIC = "fused layer-op HBM GB/s (% of peak) + µs/layer-chain, Qwen3 shapes, 1 GPU"
D = 128
THETA = 1e6
EPS = 1e-6
VOCAB = 151936

WORKLOADS = {
    "qwen3-8b-prefill": dict(T=8192, H=4096, nq=32, nk=8, I=12288, layers=36, positions="sequential", pmax=8192),
    "qwen3-0.6b-prefill": dict(T=2048, H=1024, nq=16, nk=8, I=3072, layers=28, positions="sequential", pmax=2048),
    "qwen3-4b-decode-b64": dict(T=64, H=2560, nq=32, nk=8, I=9728, layers=36, positions="uniform", pmax=32768,
                                gather=True),
    "qwen3-0.6b-decode": dict(T=1, H=1024, nq=16, nk=8, I=3072, layers=28, positions="uniform", pmax=4096,
                              gather=True),
}
HEADLINE = "qwen3-8b-prefill"
OPS = ["rmsnorm", "qknorm_rope", "add_rmsnorm", "silu_mul", "residual_add"]
# the kernel each op launches at the workload shapes: (name fragment, template fragment)
OP_KERNELS = {"rmsnorm": ("rmsnorm_row_kernel", "false, false, "), "qknorm_rope": ("qknorm_rope128_w8_kernel", ""),
              "add_rmsnorm": ("rmsnorm_row_kernel", "true, false, "), "silu_mul": ("silu_mul_vec_kernel", ""),
              "residual_add": ("residual_add_vec_kernel", ""), "layer_ops": ("layer_ops_kernel", "")}
PROFILES = os.path.join(ROOT, "profiles")
# The counter runs behind profiles/pmc_traffic_<workload>.txt (run from the repo root):
# one counter per run over `bench.py <args>`, and the same counter over a plain
# 1 GiB device copy for the calibration.
def pmc_commands(fetch_dir, write_dir, copy_fetch_dir, copy_write_dir, args):
    run = lambda c, d, a: f"rocprofv3 --pmc {c} --output-format csv -d {d} -o r -- python bench.py {a}"
    return [run("FETCH_SIZE", fetch_dir, args), run("WRITE_SIZE", write_dir, args),
            run("FETCH_SIZE", copy_fetch_dir, "--calibrate-copy"), run("WRITE_SIZE", copy_write_dir, "--calibrate-copy")]


COPY_BYTES = 1 << 30  # read and written by --calibrate-copy


def op_bytes(w):
    """Algorithmic (compulsory) HBM bytes per launch of each op: every input
    read once, every output written once (fp32 activations; gammas ignored)."""
    T, H, I, nh = w["T"], w["H"], w["I"], w["nq"] + w["nk"]
    return {
        "rmsnorm": 2 * T * H * 4,                                   # read x, write xn
        "qknorm_rope": 2 * T * nh * D * 4 + T * (D // 2) * 2 * 4,   # q, k in place + cos/sin rows
        "add_rmsnorm": 4 * T * H * 4,                               # read x, y; write x, xn
        "silu_mul": 3 * T * I * 4,                                  # read g, u; write h
        "residual_add": 3 * T * H * 4,                              # read x, y; write x
    }


def layer_ops_bytes(w):
    """Compulsory HBM bytes of one anelm_layer_ops launch: x read and written
    once (it stays in registers through the three x ops), attn and mlp read,
    both norms' outputs written, q/k in place with their cos/sin rows, g and
    u read and h written."""
    T, H, I, nh = w["T"], w["H"], w["I"], w["nq"] + w["nk"]
    return 6 * T * H * 4 + 2 * T * nh * D * 4 + T * (D // 2) * 2 * 4 + 3 * T * I * 4


def gather_bytes(w):
    return w["T"] * w["H"] * (2 + 4) if w.get("gather") else 0   # fp16 row in, fp32 row out


def qwen3_8b_tensor_sizes():
    H, I, V, L = 4096, 12288, VOCAB, 36
    sizes = [V * H, V * H, H]
    for _ in range(L):
        sizes += [H * H, 1024 * H, 1024 * H, H * H, I * H, I * H, H * I, H, H, D, D]
    return sizes


def capture(fn):
    """Record fn's launches (on torch's current stream) into a HIP graph."""
    import torch

    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        fn()
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        fn()
    torch.cuda.synchronize()
    return g


def time_region(fn, reps):
    """Average ms per call of fn over reps calls, HIP events on the current stream."""
    import torch

    s, e = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    s.record()
    for _ in range(reps):
        fn()
    e.record()
    torch.cuda.synchronize()
    return s.elapsed_time(e) / reps


ROTATE_SETS = 4   # residual-stream / output buffer sets the prefill chains rotate over


class Chain:
    """Device buffers of one op-chain workload and its per-layer launches.

    With `sets` > 1 the residual stream x and the outputs xn, h rotate over
    that many buffer sets from layer to layer (layer l uses set l % sets), so
    no layer finds what the layer before it wrote still in the 256 MB
    Infinity Cache: every layer's traffic then comes from HBM.  With one set
    x is carried through all layers, as a model does, and at the 8B prefill
    shape part of each layer's x, xn and h is then served from that cache."""

    def __init__(self, w, seed=0, sets=1):
        import torch

        import anelm

        self.w, self.hip = w, anelm
        T, H, I, nq, nk, L = w["T"], w["H"], w["I"], w["nq"], w["nk"], w["layers"]
        g = torch.Generator(device="cuda").manual_seed(seed)
        rn = lambda *s: torch.randn(*s, generator=g, device="cuda", dtype=torch.float32)
        gamma = lambda n: (1.0 + 0.02 * rn(n)).to(torch.float16)
        self.sets = [(rn(T, H), torch.empty(T, H, device="cuda"), torch.empty(T, I, device="cuda"))
                     for _ in range(sets)]
        self.x, self.xn, self.h = self.sets[0]
        self.layers = [dict(attn=rn(T, H), mlp=rn(T, H), q=rn(T, nq * D), k=rn(T, nk * D), g=rn(T, I), u=rn(T, I),
                            w_in=gamma(H), w_post=gamma(H), wq=gamma(D), wk=gamma(D)) for _ in range(L)]
        if w["positions"] == "sequential":
            self.pos = torch.arange(T, device="cuda", dtype=torch.int32)
        else:
            self.pos = torch.randint(0, w["pmax"], (T,), generator=g, device="cuda", dtype=torch.int32)
        self.cos = torch.empty(16384, D // 2, device="cuda")
        self.sin = torch.empty(16384, D // 2, device="cuda")
        anelm.rope_table(self.cos, self.sin, THETA)
        self.table = None
        if w.get("gather"):  # embedding table [151936, H] fp16 ~N(0, 0.02) and the step's token ids
            self.table = (0.02 * rn(VOCAB, H)).to(torch.float16)
            self.ids = torch.randint(0, VOCAB, (T,), generator=g, device="cuda", dtype=torch.int32)

    def op(self, name, Ld):
        hip, w = self.hip, self.w
        if name == "rmsnorm":
            hip.rmsnorm(self.xn, self.x, Ld["w_in"], EPS)
        elif name == "qknorm_rope":
            hip.qknorm_rope(Ld["q"], Ld["k"], Ld["wq"], Ld["wk"], self.pos, self.cos, self.sin, THETA, EPS,
                            nq=w["nq"], nk=w["nk"])
        elif name == "add_rmsnorm":
            hip.add_rmsnorm(self.x, Ld["attn"], self.xn, Ld["w_post"], EPS)
        elif name == "silu_mul":
            hip.silu_mul(self.h, Ld["g"], Ld["u"])
        else:
            hip.residual_add(self.x, Ld["mlp"])

    def use_set(self, li):
        self.x, self.xn, self.h = self.sets[li % len(self.sets)]

    def step(self, rotate=True):
        if self.table is not None:
            self.use_set(0)
            self.hip.embed_gather(self.x, self.table, self.ids)
        for li, Ld in enumerate(self.layers):
            self.use_set(li if rotate else 0)
            for name in OPS:
                self.op(name, Ld)
        self.use_set(0)


def prefill(w):
    return w["positions"] == "sequential"


def measure_chain(w, steps, warmup, per_op, chain_only=False, op_steps=None):
    """The op chain over all layers, graph-replayed.  Prefill workloads
    rotate x, xn and h over ROTATE_SETS sets across layers and also report
    the chain with one x carried through all layers (`carried_x`, which
    includes Infinity-Cache reuse); decode workloads carry x, as a decode
    step does (their buffers are cache-sized anyway).  With per_op, each op
    alone over all layers (one graph per op, `op_steps` timed replays after
    `warmup`): the op-major step whose time is the sum of the five."""
    import torch

    rotate = prefill(w)
    chain = Chain(w, sets=ROTATE_SETS if rotate else 1)
    ob = op_bytes(w)
    layer_bytes = sum(ob.values())
    chain_bytes = layer_bytes * w["layers"] + gather_bytes(w)

    def run(rot):
        g = capture(lambda: chain.step(rotate=rot))
        for _ in range(warmup):
            g.replay()
        ms = time_region(g.replay, steps)
        del g
        return dict(ms_per_step=round(ms, 4), us_per_layer_chain=round(ms * 1e3 / w["layers"], 3),
                    GBps=round(chain_bytes / ms / 1e6, 1), frac=round(chain_bytes / ms / 1e6 / HBM_PEAK_GBPS, 4),
                    tokens_per_s=round(w["T"] / (ms / 1e3), 1))

    r = run(rotate)
    r["chain_bytes"] = chain_bytes
    r["buffer_sets"] = len(chain.sets)
    if rotate and not chain_only:
        r["carried_x"] = dict(run(False), note="one x/xn/h carried through all layers: includes Infinity-Cache "
                                              "reuse of what the previous layer wrote")
    if not chain_only:
        # the same five ops per layer as one anelm_layer_ops launch (x kept in
        # registers through its three ops); GB/s over that launch's own bytes
        T, H = w["T"], w["H"]
        xn_in = [torch.empty(T, H, device="cuda") for _ in chain.sets]

        def one_launch():
            if chain.table is not None:
                chain.use_set(0)
                chain.hip.embed_gather(chain.x, chain.table, chain.ids)
            for li, Ld in enumerate(chain.layers):
                si = li % len(chain.sets) if rotate else 0
                chain.use_set(si)
                chain.hip.layer_ops(chain.x, xn_in[si], chain.xn, Ld["attn"], Ld["mlp"], Ld["q"], Ld["k"], chain.h,
                                    Ld["g"], Ld["u"], Ld["w_in"], Ld["w_post"], Ld["wq"], Ld["wk"], chain.pos,
                                    chain.cos, chain.sin, THETA, EPS, nq=w["nq"], nk=w["nk"])
            chain.use_set(0)
        g1 = capture(one_launch)
        for _ in range(warmup):
            g1.replay()
        ms1 = time_region(g1.replay, steps)
        del g1
        ob1 = layer_ops_bytes(w) * w["layers"] + gather_bytes(w)
        r["one_launch_per_layer"] = dict(
            ms_per_step=round(ms1, 4), us_per_layer_chain=round(ms1 * 1e3 / w["layers"], 3),
            tokens_per_s=round(w["T"] / (ms1 / 1e3), 1), bytes=ob1, GBps=round(ob1 / ms1 / 1e6, 1),
            frac=round(ob1 / ms1 / 1e6 / HBM_PEAK_GBPS, 4),
            note="anelm_layer_ops: the five ops of a layer in one launch, outputs bit-identical to the five "
                 "launches (tests/test_gpu_layer_ops.py runs it at this shape); bytes = that launch's own "
                 "compulsory traffic (x read and written once)")
        # the faster of the two tested ways to run the chain, by time per step
        fast = min((("five_launches", r["ms_per_step"]), ("one_launch_per_layer", ms1)), key=lambda p: p[1])
        r["fastest_path"] = fast[0]
        del xn_in
    if per_op:
        # Each op alone over all layers, x, xn and h rotating as in the
        # chain: no launch reads or rewrites what the launch before it left
        # in the 256 MB Infinity Cache (one op's launch touches >= 256 MB at
        # the 8B prefill shapes).
        if not rotate:
            T, H, I = w["T"], w["H"], w["I"]
            chain.sets += [(torch.randn(T, H, device="cuda"), torch.empty(T, H, device="cuda"),
                            torch.empty(T, I, device="cuda")) for _ in range(ROTATE_SETS - 1)]

        def alone(name):
            for li, Ld in enumerate(chain.layers):
                chain.use_set(li)
                chain.op(name, Ld)
            chain.use_set(0)

        ops = {}
        for name in OPS:
            go = capture(lambda: alone(name))
            for _ in range(max(warmup, 1)):
                go.replay()
            ms_all = time_region(go.replay, op_steps or (10 if w["T"] >= 1024 else 20))
            t = ms_all / len(chain.layers)
            ops[name] = dict(us=round(t * 1e3, 2), GBps=round(ob[name] / t / 1e6, 1),
                             frac=round(ob[name] / t / 1e6 / HBM_PEAK_GBPS, 4), bytes=ob[name],
                             ms_all_layers=ms_all)
            del go
        r["ops"] = ops
    del chain
    torch.cuda.empty_cache()
    return r


def measure_sampler(hip, steps, rows=64, vocab=VOCAB, freq=0.1, calls=8):
    """Logits [rows, 151936] ~N(0,3), history [rows, 256], rep 1.2, T 0.6,
    freq 0.1 (the reference default) or as given.  One graph holds `calls`
    sampler calls on distinct logits and outputs (at 64 rows more than the
    Infinity Cache holds), as a decode loop's graph would hold the sampler;
    us is per call.  one_call_per_graph: the same with a graph launch per call."""
    import torch

    g = torch.Generator(device="cuda").manual_seed(21)
    logits = [3.0 * torch.randn(rows, vocab, generator=g, device="cuda") for _ in range(calls)]
    hist = torch.randint(0, vocab, (rows, 256), generator=g, device="cuda", dtype=torch.int32)
    r = [torch.rand(rows, generator=g, device="cuda") for _ in range(calls)]
    ids = torch.empty(calls, rows, dtype=torch.int32, device="cuda")
    probs = [torch.empty(rows, vocab, device="cuda") for _ in range(calls)]
    ws = torch.empty(hip.sample_workspace_size(rows, vocab), dtype=torch.uint8, device="cuda")
    p = hip.SamplingParams(frequency_penalty=freq)
    byt = 2 * rows * vocab * 4
    out = {}
    for n, key in ((calls, "many"), (1, "one")):
        gr = capture(lambda: [hip.sample(ids[i], probs[i], logits[i], hist, None, p, r[i], ws) for i in range(n)])
        gr.replay()
        ms = time_region(gr.replay, steps) / n
        out[key] = ms
        del gr
    ms = out["many"]
    return dict(us=round(ms * 1e3, 2), GBps=round(byt / ms / 1e6, 1), frac=round(byt / ms / 1e6 / HBM_PEAK_GBPS, 4),
                rows_per_s=round(rows / (ms / 1e3), 1), bytes=byt, calls_per_graph=calls,
                one_call_per_graph_us=round(out["one"] * 1e3, 2),
                note="algorithmic bytes = logits read once + probabilities written once; us per call in a graph of "
                     f"{calls} calls on distinct inputs (one_call_per_graph_us: a graph launch per call)")


def measure_convert(hip, reps=3):
    """bf16->fp16 of the 8,190,735,360-parameter Qwen3-8B set: one call over the
    contiguous set, one call per tensor (399 launches, graph-replayed), and
    the tensors through the multi-tensor call (4 launches)."""
    import torch

    sizes = qwen3_8b_tensor_sizes()
    n = sum(sizes)
    src = torch.empty(n, dtype=torch.int16, device="cuda")
    g = torch.Generator(device="cuda").manual_seed(11)
    step = 1 << 28
    for i in range(0, n, step):
        m = min(step, n - i)
        src[i:i + m] = ((torch.randn(m, generator=g, device="cuda") * 0.02).view(torch.int32) >> 16).to(torch.int16)
    dst = torch.empty_like(src)
    byt = 4 * n
    one = lambda: hip.bf16_to_f16(dst, src)
    one()
    ms_one = time_region(one, reps)
    views = []
    off = 0
    for m in sizes:
        views.append((dst[off:off + m], src[off:off + m]))
        off += m
    gr = capture(lambda: [hip.bf16_to_f16(d, s) for d, s in views])
    gr.replay()
    ms_per = time_region(gr.replay, reps)
    dl, sl = [d for d, _ in views], [s for _, s in views]
    multi = lambda: hip.bf16_to_f16_multi(dl, sl)
    multi()
    ms_multi = time_region(multi, reps)
    del src, dst, views, gr, dl, sl
    torch.cuda.empty_cache()
    f = lambda ms: dict(ms=round(ms, 4), GBps=round(byt / ms / 1e6, 1), frac=round(byt / ms / 1e6 / HBM_PEAK_GBPS, 4))
    return dict(params=n, bytes=byt, contiguous_set=f(ms_one), per_tensor=dict(f(ms_per), launches=len(sizes)),
                per_tensor_batched=dict(f(ms_multi), launches=-(-len(sizes) // 128),
                                        note="anelm_bf16_to_f16_multi: the same tensors, up to 128 per launch"))


ATTN_WORKLOADS = {
    # Qwen3-8B attention shapes over the reference's 2048-row KV ring
    # (models/llm/qwen3.h:56), every ring full and wrapped at a random start
    "attention-qwen3-8b-decode-b64": dict(B=64, nq=32, nk=8, D=128, cap=2048),
    "attention-qwen3-8b-decode-b1": dict(B=1, nq=32, nk=8, D=128, cap=2048),
}


def attn_bytes(w):
    """K and V rows of every live position read once, q read and out written once."""
    return w["B"] * (w["cap"] * w["nk"] * w["D"] * 4 * 2 + 2 * w["nq"] * w["D"] * 4)


def measure_attention(hip, w, steps, layers=8):
    """One decode step's attention over `layers` distinct layers' KV rings
    (so the caches come from HBM), graph-replayed."""
    import torch

    B, nq, nk, D, cap = w["B"], w["nq"], w["nk"], w["D"], w["cap"]
    g = torch.Generator(device="cuda").manual_seed(31)
    rn = lambda *s: torch.randn(*s, generator=g, device="cuda")
    lay = [dict(k=rn(B, cap, nk * D), v=rn(B, cap, nk * D), q=rn(B, nq * D)) for _ in range(layers)]
    start = torch.randint(0, cap, (B,), generator=g, device="cuda", dtype=torch.int32)
    length = torch.full((B,), cap, device="cuda", dtype=torch.int32)
    out = torch.empty(B, nq * D, device="cuda")
    ws = torch.zeros(max(hip.gqa_workspace_size(B, nq, nk, D, cap), 1), dtype=torch.uint8, device="cuda")
    call = lambda: [hip.gqa_attention(out, L["q"], L["k"], L["v"], start, length, nq, nk, D, ws) for L in lay]
    gr = capture(call)
    gr.replay()
    ms = time_region(gr.replay, steps) / layers
    byt = attn_bytes(w)
    del lay, gr
    torch.cuda.empty_cache()
    return dict(us=round(ms * 1e3, 2), GBps=round(byt / ms / 1e6, 1), frac=round(byt / ms / 1e6 / HBM_PEAK_GBPS, 4),
                bytes=byt, tokens_per_s=round(B / (ms / 1e3), 1),
                note="per layer; algorithmic bytes = full K and V rings read once + q and out")


DN_WORKLOADS = {
    # Qwen3.5-0.8B linear-attention layer shapes (models/llm/qwen3_5.h:40-44): 16 key and
    # 16 value heads of 128, conv kernel 4 over 2*2048 + 2048 channels
    "deltanet-qwen3.5-0.8b-decode-b64": dict(B=64, nvh=16, nkh=16, kd=128, vd=128, K=4),
    "deltanet-qwen3.5-0.8b-decode-b1": dict(B=1, nvh=16, nkh=16, kd=128, vd=128, K=4),
}


def dn_bytes(w):
    """Per layer and token: the delta-rule states read and written once (the
    dominant term), conv rings read and written, q/k/v/z/x/y activations and
    the conv weights once; for the one-launch layer, the same less the conv
    output's store and re-read."""
    B, nvh, nkh, kd, vd, K = w["B"], w["nvh"], w["nkh"], w["kd"], w["vd"], w["K"]
    ch = 2 * nkh * kd + nvh * vd
    state = B * nvh * kd * vd * 4 * 2
    conv = B * ch * (K - 1) * 4 * 2 + ch * K * 4 + B * ch * 4 * 2
    acts = B * (2 * nkh * kd * 4 * 2 + nvh * vd * 4 * 3 + nvh * vd * 4 * 2)
    # one launch: the conv's q, k, v stay on chip (not written, not re-read)
    one = state + conv - B * ch * 4 + B * (nvh * vd * 4 * 2)
    return dict(ssm_step=state + B * (2 * nkh * kd + 2 * nvh * vd) * 4, layer=state + conv + acts, layer_one_call=one)


def measure_deltanet(hip, w, steps, layers=8):
    """One decode step of the linear-attention layer ops (qwen3_5.cpp:513-549:
    conv1d_update, SiLU, L2-normalised and scaled q, L2-normalised k, the
    delta-rule step, gated RMSNorm) over `layers` distinct layers' states,
    graph-replayed: through the two fused calls and as six separate calls;
    plus the state step alone."""
    import torch

    B, nvh, nkh, kd, vd, K = w["B"], w["nvh"], w["nkh"], w["kd"], w["vd"], w["K"]
    ch = 2 * nkh * kd + nvh * vd
    g = torch.Generator(device="cuda").manual_seed(41)
    rn = lambda *s: torch.randn(*s, generator=g, device="cuda")
    lay = [dict(S=0.05 * rn(B, nvh, kd, vd), conv=rn(B, ch, K - 1), cw=rn(ch, K), pos=torch.zeros(B, dtype=torch.int32, device="cuda"),
                decay=torch.rand(B, nvh, generator=g, device="cuda"), beta=torch.rand(B, nvh, generator=g, device="cuda"),
                nw=1.0 + 0.02 * rn(vd), hpos=torch.zeros(B, nvh, dtype=torch.int32, device="cuda"))
           for _ in range(layers)]
    x = rn(B, ch)
    z = rn(B, nvh * vd)
    mixed = torch.empty(B, ch, device="cuda")
    y = torch.empty(B, nvh * vd, device="cuda")
    out = torch.empty(B, nvh * vd, device="cuda")
    qs = float(1.0 / (kd ** 0.5))

    def layer_separate(L):
        hip.conv1d_update(mixed, L["conv"], L["pos"], x, L["cw"])               # :513
        hip.silu(mixed)                                                         # :514
        hip.l2_normalize(mixed[:, :nkh * kd], qs, heads=nkh)                     # :528, :530-531
        hip.l2_normalize(mixed[:, nkh * kd:2 * nkh * kd], 1.0, heads=nkh)        # :529
        hip.ssm_step(y, L["S"], mixed[:, :nkh * kd], mixed[:, nkh * kd:2 * nkh * kd], mixed[:, 2 * nkh * kd:],
                     L["decay"], L["beta"], nkh)                                # :533-542
        hip.rmsnorm_gated(out, y, z, L["nw"], heads=nvh)                         # :545-549

    def layer_one(L):   # the same in one launch (ring positions per head)
        hip.conv_ssm_step_gated_norm(out, L["S"], L["conv"], L["hpos"], x, L["cw"], L["decay"], L["beta"], z,
                                     L["nw"], qs)  # :513-549

    def layer(L):   # the same in two launches
        hip.conv1d_silu_l2norm(mixed, L["conv"], L["pos"], x, L["cw"], nkh, qs)  # :513-531
        hip.ssm_step_gated_norm(out, L["S"], mixed[:, :nkh * kd], mixed[:, nkh * kd:2 * nkh * kd],
                                mixed[:, 2 * nkh * kd:], L["decay"], L["beta"], z, L["nw"], nkh)  # :533-549

    gr = capture(lambda: [layer(L) for L in lay])
    gr.replay()
    ms = time_region(gr.replay, steps) / layers
    g6 = capture(lambda: [layer_separate(L) for L in lay])
    g6.replay()
    ms6 = time_region(g6.replay, steps) / layers
    ms1 = None
    if nvh == nkh and kd == 128 and vd == 128 and K == 4:
        g1 = capture(lambda: [layer_one(L) for L in lay])
        g1.replay()
        ms1 = time_region(g1.replay, steps) / layers
        del g1
    gs = capture(lambda: [hip.ssm_step(y, L["S"], mixed[:, :nkh * kd], mixed[:, nkh * kd:2 * nkh * kd],
                                       mixed[:, 2 * nkh * kd:], L["decay"], L["beta"], nkh) for L in lay])
    gs.replay()
    ms_s = time_region(gs.replay, steps) / layers
    b = dn_bytes(w)
    del lay, gr, gs, g6
    torch.cuda.empty_cache()
    f = lambda byt, ms: dict(us=round(ms * 1e3, 2), GBps=round(byt / ms / 1e6, 1),
                             frac=round(byt / ms / 1e6 / HBM_PEAK_GBPS, 4), bytes=byt)
    r = dict(layer=dict(f(b["layer"], ms), tokens_per_s=round(B / (ms / 1e3), 1)),
             layer_six_calls=f(b["layer"], ms6), ssm_step=f(b["ssm_step"], ms_s),
             note="per layer; algorithmic bytes = delta-rule states read+written once, conv rings, activations; "
                  "layer = anelm_conv1d_silu_l2norm + anelm_ssm_step_gated_norm, layer_one_call = "
                  "anelm_conv_ssm_step_gated_norm, layer_six_calls = the six separate ops")
    if ms1 is not None:
        r["layer_one_call"] = dict(f(b["layer_one_call"], ms1), tokens_per_s=round(B / (ms1 / 1e3), 1))
    return r


def cpu_attention(w, target_s):
    """The oracle's gqa_attention (heads in parallel, as the reference runs
    them) for one sequence, repeated for about target_s seconds."""
    import numpy as np

    oracle = _oracle()
    nq, nk, D, cap = w["nq"], w["nk"], w["D"], w["cap"]
    rng = np.random.default_rng(4)
    kc = rng.standard_normal((cap, nk * D), dtype=np.float32)
    vc = rng.standard_normal((cap, nk * D), dtype=np.float32)
    q = rng.standard_normal(nq * D, dtype=np.float32)
    t0 = time.perf_counter()
    done = 0
    while True:
        oracle.gqa_attention(q, kc, vc, nq, nk, D, 17, cap)
        done += 1
        el = time.perf_counter() - t0
        if el >= target_s:
            break
    per_seq = el / done
    byt = attn_bytes(dict(w, B=1))
    return dict(us_per_sequence=round(per_seq * 1e6, 1), GBps=round(byt / per_seq / 1e9, 2),
                cores=oracle.max_threads(), kind="port",
                sample=f"{done} single-sequence calls (capacity {cap}, full ring) on {oracle.max_threads()} threads")


def qwen3_06b_tensors():
    """Tensor names and shapes of a Qwen3-0.6B checkpoint (tied LM head)."""
    H, I, L = 1024, 3072, 28
    t = {"model.embed_tokens.weight": (VOCAB, H), "model.norm.weight": (H,)}
    for l in range(L):
        p = f"model.layers.{l}."
        t.update({p + "self_attn.q_proj.weight": (2048, H), p + "self_attn.k_proj.weight": (1024, H),
                  p + "self_attn.v_proj.weight": (1024, H), p + "self_attn.o_proj.weight": (H, 2048),
                  p + "self_attn.q_norm.weight": (D,), p + "self_attn.k_norm.weight": (D,),
                  p + "mlp.gate_proj.weight": (I, H), p + "mlp.up_proj.weight": (I, H),
                  p + "mlp.down_proj.weight": (H, I), p + "input_layernorm.weight": (H,),
                  p + "post_attention_layernorm.weight": (H,)})
    return t


def make_blob_checkpoint(path):
    """A synthetic bf16 safetensors file of Qwen3-0.6B shapes (~1.2 GB)."""
    import torch
    from safetensors.torch import save_file

    g = torch.Generator().manual_seed(13)
    ts = {n: (0.02 * torch.randn(*s, generator=g)).bfloat16() for n, s in qwen3_06b_tensors().items()}
    save_file(ts, path)
    return sum(t.numel() for t in ts.values())


def measure_blobs(hip, workdir, reps=2):
    """The `convert` command (core/safetensors.cpp:345-383) on a Qwen3-0.6B-shaped
    checkpoint: parse, convert on the GPU, write every blob; wall clock
    including the file writes (best of reps)."""
    import shutil

    src = os.path.join(workdir, "qwen3-0.6b-shaped.safetensors")
    n = make_blob_checkpoint(src)
    best = None
    for r in range(reps):
        out = os.path.join(workdir, f"blobs{r}")
        t0 = time.perf_counter()
        k = hip.write_ane_blobs(src, out)
        el = time.perf_counter() - t0
        best = el if best is None else min(best, el)
        shutil.rmtree(out, ignore_errors=True)
    return src, dict(seconds=round(best, 3), params=n, blobs=k, params_per_s=round(n / best, 1),
                     GBps_in_out=round(4 * n / best / 1e9, 2),
                     note="wall clock of anelm_write_ane_blobs incl. page-cache reads and file writes")


Q3_WORKLOADS = {
    # one decode step of a Qwen3-0.6B-shaped model (random weights) for B
    # sequences: every layer op, the attention over rings of capacity 2048
    # and the fp16 projections (the reference's ANE contractions) with the LM
    # head.  The rings start empty (a few dozen rows by the timed steps) or,
    # with ctx, hold that many rows from earlier steps.
    "qwen3-0.6b-decode-step-b1": dict(B=1),
    "qwen3-0.6b-decode-step-b64": dict(B=64),
    "qwen3-0.6b-decode-step-b1-ctx1024": dict(B=1, ctx=1024),
    "qwen3-0.6b-decode-step-b64-ctx1024": dict(B=64, ctx=1024),
}
Q3_06B = dict(hidden=1024, layers=28, n_q_heads=16, n_kv_heads=8, head_dim=D, intermediate=3072, vocab=VOCAB)


def q3_weight_bytes():
    """fp16 projection and LM-head bytes one step reads (the norms and the
    gathered embedding rows are negligible)."""
    c = Q3_06B
    per_layer = ((c["n_q_heads"] + 2 * c["n_kv_heads"]) * D * c["hidden"] + c["hidden"] * c["n_q_heads"] * D +
                 3 * c["intermediate"] * c["hidden"])
    return 2 * (c["layers"] * per_layer + c["vocab"] * c["hidden"])


def measure_qwen3(hip, src, w, steps=30):
    """Graph-replayed decode steps (positions advance inside the graph) from
    empty rings, or after w["ctx"] eager steps; tokens/s = B x steps / time."""
    import torch

    B = w["B"]
    cfg = hip.Qwen3Config(*[Q3_06B[k] for k in ("hidden", "layers", "n_q_heads", "n_kv_heads", "head_dim",
                                                 "intermediate", "vocab")], THETA, EPS)
    model = hip.Qwen3Model(src, cfg, max_batch=B, kv_capacity=2048)
    g = torch.Generator(device="cuda").manual_seed(17)
    ids = torch.randint(0, VOCAB, (B,), generator=g, device="cuda", dtype=torch.int32)
    pos = torch.zeros(B, dtype=torch.int32, device="cuda")
    logits = torch.empty(B, VOCAB, device="cuda")

    def step():
        model.forward(ids, pos, logits)
        pos.add_(1)
    for _ in range(max(1, w.get("ctx", 0))):
        step()
    gr = capture(step)
    for _ in range(3):
        gr.replay()
    ms = time_region(gr.replay, steps)
    byt = q3_weight_bytes()
    # K and V rows each timed step reads: the rings hold ctx rows (at least
    # one step) + 1 (capture's run) + 3 (warm replays), plus one more per step
    c = Q3_06B
    rows = max(1, w.get("ctx", 0)) + 4 + (steps + 1) / 2
    kv = int(c["layers"] * B * rows * c["n_kv_heads"] * D * 4 * 2)
    del gr
    model.close()
    torch.cuda.empty_cache()
    return dict(ms_per_step=round(ms, 4), tokens_per_s=round(B / (ms / 1e3), 1),
                weight_GBps=round(byt / ms / 1e6, 1), weight_frac=round(byt / ms / 1e6 / HBM_PEAK_GBPS, 4),
                weight_bytes=byt, steps=steps,
                ring_rows=f"{w.get('ctx', 0)}+ (capacity 2048)", kv_bytes=kv,
                total_GBps=round((byt + kv) / ms / 1e6, 1), total_frac=round((byt + kv) / ms / 1e6 / HBM_PEAK_GBPS, 4),
                note="weight_GBps = fp16 projection + LM-head bytes / step time; ring_rows = rows in each ring when "
                     "the timed steps start; total_GBps adds the K and V rows the attention reads (kv_bytes, "
                     "averaged over the timed steps)")


def cpu_qwen3(src, steps=2):
    """The oracle's decode step (one sequence) on the same checkpoint."""
    oracle = _oracle()
    t = {k: v[2] for k, v in oracle.read_safetensors(src).items()}
    c = Q3_06B
    cfg = oracle.Qwen3Config(c["hidden"], c["layers"], c["n_q_heads"], c["n_kv_heads"], c["head_dim"],
                             c["intermediate"], c["vocab"], THETA, EPS)
    m = oracle.Qwen3(cfg, t, 1, 2048)
    import numpy as np

    m.forward(np.array([1], np.int32), np.array([0], np.int32))
    t0 = time.perf_counter()
    for s in range(steps):
        m.forward(np.array([7 + s], np.int32), np.array([1 + s], np.int32))
    el = (time.perf_counter() - t0) / steps
    return dict(ms_per_step=round(el * 1e3, 1), tokens_per_s=round(1 / el, 2), cores=oracle.max_threads(),
                kind="port", sample=f"{steps} single-sequence steps of the oracle's decode step (fp64 projections)")


def cpu_blobs(src, workdir):
    import shutil

    oracle = _oracle()
    out = os.path.join(workdir, "blobs_cpu")
    t0 = time.perf_counter()
    k = oracle.write_ane_blobs(src, out)
    el = time.perf_counter() - t0
    shutil.rmtree(out, ignore_errors=True)
    return dict(seconds=round(el, 3), blobs=k, cores=oracle.max_threads(), kind="port",
                sample="the oracle's write_ane_blobs (numpy reader, C convert) on the same file")


# ------------------------------------------------------------------ CPU baseline

def _oracle():
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import oracle

    return oracle


def cpu_chain(w, target_s, max_tokens=512, layers=4, threads=None):
    """The oracle's per-token layer chain (looping per token as the reference
    does) on the host's cores (or `threads` of them), over a bounded sample:
    up to max_tokens tokens x `layers` distinct layers of the workload's
    shapes, repeated for about target_s seconds.  Reported in the GPU
    figure's unit (algorithmic GB/s)."""
    import numpy as np

    oracle = _oracle()
    T = min(w["T"], max_tokens)
    H, I, nq, nk = w["H"], w["I"], w["nq"], w["nk"]
    rng = np.random.default_rng(5)
    rn = lambda *s: rng.standard_normal(s, dtype=np.float32)
    lay = [dict(attn=rn(T, H), mlp=rn(T, H), q=rn(T, nq * D), k=rn(T, nk * D), g=rn(T, I), u=rn(T, I))
           for _ in range(layers)]
    gam = lambda n: (1 + 0.02 * rng.standard_normal(n)).astype(np.float16).astype(np.float32)
    w_in, w_post, wq, wk = gam(H), gam(H), gam(D), gam(D)
    x, xn, h = rn(T, H), np.empty((T, H), np.float32), np.empty((T, I), np.float32)
    pos = (np.arange(T) % w["pmax"]).astype(np.int32)
    c, s = oracle.rope_table(16384, D, THETA)
    threads = threads or oracle.max_threads()
    t0 = time.perf_counter()
    passes = 0
    while True:
        for Ld in lay:
            oracle.layer_chain(T, H, nq, nk, D, I, x, xn, Ld["attn"], Ld["mlp"], Ld["q"], Ld["k"], Ld["g"], Ld["u"],
                               h, w_in, w_post, wq, wk, pos, c, s, THETA, EPS, threads)
        passes += 1
        el = time.perf_counter() - t0
        if el >= target_s:
            break
    per_layer_bytes = sum(op_bytes(dict(w, T=T)).values())
    gbps = per_layer_bytes * layers * passes / el / 1e9
    us_layer = el / (layers * passes) * (w["T"] / T) * 1e6
    return dict(value=round(gbps, 2), unit="GB/s", cores=threads, kind="port",
                us_per_layer_chain=round(us_layer, 1),
                sample=f"oracle layer chain, per-token loop as the reference, {T} tokens x {layers} distinct layers "
                       f"of the workload's shapes, {passes} passes in {el:.1f} s on {threads} OpenMP threads")


def cpu_sampler(target_s, rows=64, vocab=VOCAB, freq=0.1):
    import numpy as np

    oracle = _oracle()
    rng = np.random.default_rng(9)
    logits = rng.normal(0, 3, (rows, vocab)).astype(np.float32)
    hist = rng.integers(0, vocab, (rows, 256)).astype(np.int32)
    t0 = time.perf_counter()
    done = 0
    while True:
        oracle.sample_token(logits[done % rows], recent=hist[done % rows], r=0.5, frequency_penalty=freq)
        done += 1
        el = time.perf_counter() - t0
        if el >= target_s:
            break
    per_row = el / done
    return dict(us=round(per_row * rows * 1e6, 1), GBps=round(2 * rows * vocab * 4 / (per_row * rows) / 1e9, 2),
                cores=1, kind="port", sample=f"{done} rows of sample_token on 1 thread (the reference is single-threaded)")


def cpu_convert(target_s):
    import numpy as np

    oracle = _oracle()
    src = np.random.default_rng(3).integers(0, 65536, 1 << 26, dtype=np.uint32).astype(np.uint16)
    t0 = time.perf_counter()
    done = 0
    while True:
        oracle.bf16_to_f16(src)
        done += src.size
        el = time.perf_counter() - t0
        if el >= target_s:
            break
    return dict(GBps=round(4 * done / el / 1e9, 2), cores=oracle.max_threads(), kind="port",
                sample=f"{done} parameters in chunks of 2^26 on {oracle.max_threads()} threads")


def dropin_per_call():
    """Per-call wall time of the unchanged-caller path: ane_lm::rmsnorm at
    dim 1024 and 128 (and a layer's 40 head norms from 8 threads),
    ane_lm::sample_token at 151936, and the additive entries
    hip::qknorm_rope_qwen3 (a layer's 40 head norms + RoPE in one call),
    hip::residual_add and hip::silu_mul at the Qwen3-8B per-token sizes, each
    a synchronous host-pointer call through the drop-in layer, beside the
    oracle's single-thread CPU time of the same function
    (tests/cpp/dropin_timing.cpp, built by build())."""
    import subprocess

    exe = os.path.join(ROOT, "tests", "cpp", "dropin_timing")
    if not os.path.exists(exe):
        return dict(note="tests/cpp/dropin_timing not built")
    r = subprocess.run([exe], stdout=subprocess.PIPE, stderr=subprocess.PIPE, text=True, timeout=300)
    if r.returncode != 0:
        raise SystemExit(f"dropin_timing failed ({r.returncode}): {r.stderr[-2000:]}")
    out = json.loads(r.stdout.strip().splitlines()[-1])
    out["note"] = ("wall time per call from the host, H2D + kernels + D2H + stream sync; oracle = the same function "
                   "on one CPU thread (the reference's cost where it runs on the CPU)")
    return out


# ------------------------------------------------------------ rocprofv3 summaries

def _csv_rows(d, suffix):
    import csv
    import glob

    rows = []
    for f in sorted(glob.glob(os.path.join(d, "**", "*" + suffix), recursive=True)):
        with open(f, newline="") as fh:
            rows += list(csv.DictReader(fh))
    if not rows:
        raise SystemExit(f"no *{suffix} under {d}")
    return rows


ATTN_KERNELS = {"gqa_decode": ("gqa_decode_kernel", "")}
DN_B64 = "deltanet-qwen3.5-0.8b-decode-b64"
DN_KERNELS = {"layer_one_call": ("conv_ssm_kernel", ""), "conv_silu_l2": ("conv_silu_l2_kernel", ""),
              "ssm_step_gated": ("ssm_step_kernel", "128, 0>"), "ssm_step": ("ssm_step_kernel", "128, -1>")}


SAMPLE_KERNELS = {"stages_one_launch": ("sample_fused_kernel", ""), "stage1": ("sample_stage1_kernel", ""),
                  "stage2": ("sample_stage2_kernel", ""), "stage3": ("sample_stage3_kernel", ""),
                  "walk": ("sample_walk_kernel", "")}
SAMPLER = "sampling-64x151936"

# The 64-sequence decode step's LM head (x staged in LDS) and layer kernels
# (tiled x and W: <fp16 x, batch tiles, row tiles, steps in flight, norm,
# epilogue, waves, tiled W, tiled x>)
Q3_B64 = "qwen3-0.6b-decode-step-b64"
Q3_B64_KERNELS = {"lm_head": ("proj_lds_kernel", ""), "attention": ("gqa_decode_kernel", ""),
                  "norm_f16_tiled": ("rmsnorm_row_kernel", "false, true, true, true>"),
                  "qkv": ("proj_mfma_kernel", "<true, 2, 2, 8, false, 0, 4, true, true>"),
                  "o_proj_add": ("proj_mfma_kernel", "<true, 1, 1, 16, false, 1, 4, true, true>"),
                  "gate_up_swiglu": ("proj_mfma_kernel", "<true, 4, 2, 8, false, 5, 4, true, true>"),
                  "down_add": ("proj_mfma_kernel", "<true, 1, 1, 24, false, 1, 4, true, true>")}

# The one-sequence decode step's projections, told apart by their launch
# shapes <rows of x, rows per wave, chunks in flight, x form (0 fp32, 1 fp32
# through the fused RMSNorm, 2 fp16), epilogue>
Q3_B1 = "qwen3-0.6b-decode-step-b1"
Q3_KERNELS = {"qkv": ("proj_dot_kernel", "<1, 2, 2, 1, 0>"), "o_proj": ("proj_dot_kernel", "<1, 1, 4, 2, 1>"),
              "gate_up": ("proj_dot_kernel", "<1, 1, 2, 1, 3>"), "down": ("proj_dot_kernel", "<1, 1, 6, 2, 1>"),
              "lm_head": ("proj_dot_kernel", "<1, 4, 2, 1, 0>")}


def q3_b1_bytes():
    """fp16 weight bytes each projection of the one-sequence step reads (its
    activations are a few KB)."""
    c = Q3_06B
    H, I, qd = c["hidden"], c["intermediate"], c["n_q_heads"] * D
    return {"qkv": 2 * (qd + 2 * c["n_kv_heads"] * D) * H, "o_proj": 2 * H * qd, "gate_up": 2 * 2 * I * H,
            "down": 2 * H * I, "lm_head": 2 * c["vocab"] * H}


def q3_b64_bytes(B=64):
    """Algorithmic bytes per dispatch of the 64-sequence step's kernels: fp16
    weights once, fp16 inputs once, outputs written once (read too for the
    residual adds); the attention's K/V rows depend on the ring lengths and
    are not counted here."""
    c = Q3_06B
    H, I, qd = c["hidden"], c["intermediate"], c["n_q_heads"] * D
    qkvd = qd + 2 * c["n_kv_heads"] * D
    return {"lm_head": 2 * c["vocab"] * H + B * H * 2 + B * c["vocab"] * 4,
            "attention": 0,
            "norm_f16_tiled": B * H * 4 + B * H * 2,
            "qkv": 2 * qkvd * H + B * H * 2 + B * qkvd * 4,
            "o_proj_add": 2 * H * qd + B * qd * 2 + 2 * B * H * 4,
            "gate_up_swiglu": 2 * 2 * I * H + B * H * 2 + B * I * 2,
            "down_add": 2 * H * I + B * I * 2 + 2 * B * H * 4}


def _kernels_of(workload):
    if workload == SAMPLER:
        return SAMPLE_KERNELS
    if workload == Q3_B1:
        return Q3_KERNELS
    if workload == Q3_B64:
        return Q3_B64_KERNELS
    if workload == DN_B64:
        return DN_KERNELS
    return ATTN_KERNELS if workload in ATTN_WORKLOADS else OP_KERNELS


def _run_args(workload):
    """bench.py arguments of the run a counter summary of `workload` is made from."""
    if workload in ATTN_WORKLOADS or workload == SAMPLER:
        return f"--only {workload} --steps 1"
    if workload in (Q3_B1, Q3_B64):
        return f"--only {workload} --no-cpu"
    if workload == HEADLINE:
        return f"--workload {workload} --chain-only --no-cpu --steps 1 --warmup 0"
    return f"--only {workload} --steps 1 --warmup 0"


# SQ counters in two passes (at most 8 SQ counters per rocprofv3 --pmc run)
SQ_PASSES = [["SQ_WAVES", "SQ_WAVE_CYCLES", "SQ_BUSY_CU_CYCLES", "SQ_WAIT_ANY", "SQ_WAIT_INST_ANY",
              "SQ_INSTS_VALU", "SQ_ACTIVE_INST_VALU", "SQ_INSTS_SALU"],
             ["SQ_INSTS_VMEM_RD", "SQ_INSTS_VMEM_WR", "SQ_INSTS_LDS", "SQ_WAIT_INST_LDS", "SQ_ACTIVE_INST_ANY",
              "GRBM_GUI_ACTIVE"],
             # rocprofv3's derived metrics over the level counters (SQ_LEVEL_WAVES, SQ_INST_LEVEL_VMEM), which
             # mean nothing unless accumulated: one per pass, each takes the accumulator
             ["MeanOccupancyPerActiveCU"], ["VmemLatency"]]
N_XCC, N_SIMD = 8, 1024   # MI355X: GRBM_GUI_ACTIVE is summed over the 8 XCCs; 256 CUs x 4 SIMDs


def sq_commands(dirs, workload):
    return [f"rocprofv3 --pmc {' '.join(c)} --output-format csv -d {d} -o r -- python bench.py {_run_args(workload)}"
            for c, d in zip(SQ_PASSES, dirs)]


def sq_summary(dirs, workload=HEADLINE):
    """Text summary of the four SQ-counter runs of sq_commands(): per kernel,
    per dispatch (SQ_WAVE_CYCLES, SQ_BUSY_CU_CYCLES, SQ_WAIT_*, SQ_ACTIVE_INST_*
    count quad-cycles; GRBM_GUI_ACTIVE counts cycles on each of the 8 XCCs):
      waves/CU    = 4 * SQ_WAVE_CYCLES / (kernel_cyc * 256 CUs)  (mean resident waves per CU over the
                    dispatch, of 32: the numerator of rocprofv3's OccupancyPercent)
      occ_rocprof = MeanOccupancyPerActiveCU             (rocprofv3's accumulated SQ_LEVEL_WAVES over
                    SQ_BUSY_CU_CYCLES, which counts each SIMD of a busy CU: a per-SIMD figure, of 8)
      wave_cyc    = 4 * SQ_WAVE_CYCLES / SQ_WAVES        (mean wave lifetime, cycles)
      wait        = SQ_WAIT_ANY / SQ_WAVE_CYCLES         (share of wave time waiting on memory or dependencies)
      issue_wait  = SQ_WAIT_INST_ANY / SQ_WAVE_CYCLES    (share of wave time waiting for an issue slot)
      vmem_lat    = VmemLatency                          (mean cycles a vector memory instruction is in flight)
      valu_util   = 4 * SQ_ACTIVE_INST_VALU / (1024 SIMDs * GRBM_GUI_ACTIVE / 8)  (VALU busy share of the chip)
      kernel_cyc  = GRBM_GUI_ACTIVE / 8"""
    cm = [_counter_means(d) for d in dirs]
    kernels = _kernels_of(workload)
    lines = [f"# SQ counters per dispatch, workload {workload} (rocprofv3 --pmc, four passes)", "#",
             "# commands (from the repo root):"] + [
             f"#   {c}" for c in sq_commands(dirs, workload)] + [
             f"#   python bench.py --workload {workload} --sq-summary {' '.join(dirs)}", "#",
             "# SQ_WAVE_CYCLES, SQ_BUSY_CU_CYCLES, SQ_WAIT_ANY, SQ_WAIT_INST_ANY, SQ_ACTIVE_INST_VALU count quad-cycles;",
             "# GRBM_GUI_ACTIVE counts cycles on each of the 8 XCCs.",
             "# waves/CU = 4*SQ_WAVE_CYCLES/(kernel cyc*256 CUs) (mean resident waves per CU over the dispatch, of 32); "
             "occ_rocprof = MeanOccupancyPerActiveCU (accumulated SQ_LEVEL_WAVES/SQ_BUSY_CU_CYCLES, per SIMD, of 8);",
             "# wave cyc = 4*SQ_WAVE_CYCLES/SQ_WAVES; wait = SQ_WAIT_ANY/SQ_WAVE_CYCLES; issue_wait = "
             "SQ_WAIT_INST_ANY/SQ_WAVE_CYCLES; vmem_lat = VmemLatency (cycles);",
             "# valu_util = 4*SQ_ACTIVE_INST_VALU/(1024*GRBM_GUI_ACTIVE/8); kernel cyc = GRBM_GUI_ACTIVE/8",
             "",
             "| op | kernel | dispatches | waves | waves/CU | occ_rocprof | kernel cyc | wave cyc | wait | issue_wait | "
             "vmem_lat | VALU/wave | valu_util | SALU/wave | LDS/wave | VMEM rd/wr per wave |",
             "|---|---|---|---|---|---|---|---|---|---|---|---|---|---|---|---|"]
    out = {}
    for op in kernels:
        v = {}
        n = 0
        kname = None
        for c in cm:
            for (k, name), (cnt, mean) in c.items():
                if _match(k, op, kernels):
                    v[name] = mean
                    n, kname = cnt, k
        need = ("SQ_WAVES", "SQ_INSTS_VMEM_RD", "GRBM_GUI_ACTIVE", "VmemLatency")
        if not all(x in v for x in need):
            continue
        wv = max(v["SQ_WAVES"], 1.0)
        wc = max(v["SQ_WAVE_CYCLES"], 1.0)
        kc = max(v["GRBM_GUI_ACTIVE"] / N_XCC, 1.0)
        d = dict(waves=round(v["SQ_WAVES"]), waves_per_cu=round(4 * v["SQ_WAVE_CYCLES"] / (kc * N_SIMD / 4), 1),
                 occ_rocprof=round(v["MeanOccupancyPerActiveCU"], 1), kernel_cycles=round(kc),
                 wave_cycles=round(4 * v["SQ_WAVE_CYCLES"] / wv), wait=round(v["SQ_WAIT_ANY"] / wc, 3),
                 issue_wait=round(v["SQ_WAIT_INST_ANY"] / wc, 3), vmem_lat=round(v["VmemLatency"]),
                 valu_per_wave=round(v["SQ_INSTS_VALU"] / wv),
                 valu_util=round(4 * v["SQ_ACTIVE_INST_VALU"] / (N_SIMD * kc), 3),
                 salu_per_wave=round(v["SQ_INSTS_SALU"] / wv), lds_per_wave=round(v["SQ_INSTS_LDS"] / wv, 1),
                 vmem_rd_per_wave=round(v["SQ_INSTS_VMEM_RD"] / wv, 1), vmem_wr_per_wave=round(v["SQ_INSTS_VMEM_WR"] / wv, 1))
        out[op] = d
        short = kname.replace("(anonymous namespace)::", "").split("(")[0].replace("void ", "")
        lines.append(f"| {op} | `{short}` | {n} | {d['waves']} | {d['waves_per_cu']} | {d['occ_rocprof']} | "
                     f"{d['kernel_cycles']} | {d['wave_cycles']} | {d['wait']} | {d['issue_wait']} | {d['vmem_lat']} | "
                     f"{d['valu_per_wave']} | {d['valu_util']} | {d['salu_per_wave']} | {d['lds_per_wave']} | "
                     f"{d['vmem_rd_per_wave']} / {d['vmem_wr_per_wave']} |")
    lines += ["", "sq_json: " + json.dumps(dict(workload=workload, per_dispatch=out))]
    return "\n".join(lines)


def _match(name, op, kernels=None):
    frag, tmpl = (kernels or OP_KERNELS)[op]
    return frag in name and tmpl in name


def _counter_means(d):
    """{(kernel name, counter): (dispatches, mean value)} of a --pmc run."""
    acc = {}
    for r in _csv_rows(d, "counter_collection.csv"):
        k = (r["Kernel_Name"], r["Counter_Name"])
        n, t = acc.get(k, (0, 0.0))
        acc[k] = (n + 1, t + float(r["Counter_Value"]))
    return {k: (n, t / n) for k, (n, t) in acc.items()}


def pmc_summary(fetch_dir, write_dir, copy_fetch_dir, copy_write_dir, workload=HEADLINE):
    """Text summary of the four counter runs of pmc_commands(): HBM bytes per
    dispatch of each op's kernel, with FETCH_SIZE / WRITE_SIZE (KiB) scaled
    by what they read for a plain 1 GiB device copy."""
    fe, wr = _counter_means(fetch_dir), _counter_means(write_dir)
    cf, cw = _counter_means(copy_fetch_dir), _counter_means(copy_write_dir)
    copy_f = max(v for (k, c), (n, v) in cf.items() if "copyBuffer" in k and c == "FETCH_SIZE")
    copy_w = max(v for (k, c), (n, v) in cw.items() if "copyBuffer" in k and c == "WRITE_SIZE")
    ff, wf = COPY_BYTES / 1024 / copy_f, COPY_BYTES / 1024 / copy_w
    kernels = _kernels_of(workload)
    run_args = _run_args(workload)
    if workload in ATTN_WORKLOADS:
        w = ATTN_WORKLOADS[workload]
        ob = {"gqa_decode": attn_bytes(w)}
    elif workload == Q3_B1:
        ob = q3_b1_bytes()
    elif workload == Q3_B64:
        ob = q3_b64_bytes()
    elif workload == DN_B64:
        w = DN_WORKLOADS[workload]
        B, nvh, nkh, kd, vd = w["B"], w["nvh"], w["nkh"], w["kd"], w["vd"]
        ch = 2 * nkh * kd + nvh * vd
        d = dn_bytes(w)
        state = B * nvh * kd * vd * 4 * 2
        ob = {"layer_one_call": d["layer_one_call"], "ssm_step": d["ssm_step"],
              "ssm_step_gated": state + B * (2 * nkh * kd + 3 * nvh * vd) * 4,   # q, k, v, z in; out
              "conv_silu_l2": B * ch * 3 * 4 * 2 + ch * 4 * 4 + B * ch * 4 * 2}  # rings, weights, x in, y out
    elif workload == SAMPLER:
        # the one launch (64 rows) reads the logits and writes the probabilities
        # once; as three launches stage 1 reads the logits, stage 2 reads them
        # again and writes exp(x - max) into the probability buffer, stage 3
        # reads that and writes the probabilities
        lv = 64 * VOCAB * 4
        ob = {"stages_one_launch": 2 * lv, "stage1": lv, "stage2": 2 * lv, "stage3": 2 * lv, "walk": 0}
    else:
        ob = dict(op_bytes(WORKLOADS[workload]), layer_ops=layer_ops_bytes(WORKLOADS[workload]))
    commands = pmc_commands(fetch_dir, write_dir, copy_fetch_dir, copy_write_dir, run_args)
    lines = [f"# HBM traffic per dispatch, workload {workload} (rocprofv3 --pmc, one counter per run)", "#",
             "# commands (from the repo root):"] + [f"#   {c}" for c in commands] + [
             f"#   python bench.py --workload {workload} --pmc-summary {fetch_dir} {write_dir} {copy_fetch_dir} "
             f"{copy_write_dir}", "#",
             f"# calibration, 1 GiB device copy: FETCH_SIZE {copy_f:.0f} KiB -> factor {ff:.4f}; "
             f"WRITE_SIZE {copy_w:.0f} KiB -> factor {wf:.4f}", "",
             "| op | kernel | dispatches | FETCH_SIZE KiB | WRITE_SIZE KiB | traffic bytes | algorithmic bytes | ratio |",
             "|---|---|---|---|---|---|---|---|"]
    traffic = {}
    for op in kernels:
        fk = [(k, v) for k, v in fe.items() if k[1] == "FETCH_SIZE" and _match(k[0], op, kernels)]
        wk = [(k, v) for k, v in wr.items() if k[1] == "WRITE_SIZE" and _match(k[0], op, kernels)]
        if not fk or not wk:
            continue
        (kname, _), (n, f) = fk[0]
        _, (_, w_) = wk[0]
        t = round((f * ff + w_ * wf) * 1024)
        traffic[op] = t
        short = kname.replace("(anonymous namespace)::", "").split("(")[0].replace("void ", "")
        ratio = f"{t / ob[op]:.4f}" if ob[op] else "-"
        lines.append(f"| {op} | `{short}` | {n} | {f:.0f} | {w_:.0f} | {t} | {ob[op]} | {ratio} |")
    lines += ["", "traffic_json: " + json.dumps(dict(workload=workload, fetch_factor=round(ff, 6),
                                                      write_factor=round(wf, 6), bytes_per_dispatch=traffic))]
    return "\n".join(lines)


def trace_summary(d, command, top=10):
    """Text summary of a --kernel-trace --stats run: the busiest kernels
    overall, then every library kernel split by launch shape (the workloads
    share kernel names, their grids tell them apart)."""
    rows = _csv_rows(d, "kernel_stats.csv")
    rows.sort(key=lambda r: -float(r["TotalDurationNs"]))
    short = lambda n: n.replace("(anonymous namespace)::", "").split("(")[0].replace("void ", "")
    lines = ["# rocprofv3 --kernel-trace --stats", "#", f"# command (from the repo root): {command}", "",
             "## busiest kernels (kernel_stats.csv)", "",
             "| kernel | calls | avg us | min us | max us | share % |", "|---|---|---|---|---|---|"]
    for r in rows[:top]:
        lines.append(f"| `{short(r['Name'])[:100]}` | {r['Calls']} | {float(r['AverageNs']) / 1e3:.2f} | "
                     f"{float(r['MinNs']) / 1e3:.2f} | {float(r['MaxNs']) / 1e3:.2f} | {float(r['Percentage']):.2f} |")
    groups = {}
    for r in _csv_rows(d, "kernel_trace.csv"):
        name = short(r["Kernel_Name"])
        if not name.startswith("anelm::"):
            continue
        grid = "x".join(r[f"Grid_Size_{c}"] for c in "XYZ")
        key = (name, grid, r["Workgroup_Size_X"])
        groups.setdefault(key, []).append((int(r["End_Timestamp"]) - int(r["Start_Timestamp"])) / 1e3)
    lines += ["", "## library kernels by launch shape (kernel_trace.csv)", "",
              "| kernel | grid (threads) | workgroup | calls | avg us | min us | max us |",
              "|---|---|---|---|---|---|---|"]
    for (name, grid, wg), t in sorted(groups.items(), key=lambda kv: -sum(kv[1])):
        lines.append(f"| `{name}` | {grid} | {wg} | {len(t)} | {sum(t) / len(t):.2f} | {min(t):.2f} | {max(t):.2f} |")
    return "\n".join(lines)


def load_traffic(workload, op):
    """Calibrated HBM bytes per dispatch of op's kernel from the committed
    counter summary, or None if there is none for this workload."""
    f = os.path.join(PROFILES, f"pmc_traffic_{workload}.txt")
    if not os.path.exists(f):
        return None
    with open(f) as fh:
        for line in fh:
            if line.startswith("traffic_json: "):
                return json.loads(line[len("traffic_json: "):])["bytes_per_dispatch"].get(op)
    return None


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--workload", default=HEADLINE, choices=sorted(WORKLOADS) + sorted(ATTN_WORKLOADS) + [SAMPLER, Q3_B1, Q3_B64, DN_B64],
                    help="op-chain workload to run (attention names only select --pmc-summary kernels)")
    ap.add_argument("--cpu-seconds", type=float, default=8.0, help="CPU time budget of the headline baseline")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--headline-only", action="store_true", help="skip the other configurations")
    ap.add_argument("--chain-only", action="store_true",
                    help="headline: only the rotating chain (no carried-x chain, no per-op timing), for counter runs")
    ap.add_argument("--calibrate-copy", action="store_true",
                    help="only time a 1 GiB device-to-device copy (reference for rocprof byte counters)")
    ap.add_argument("--only", default=None, help="measure only this named configuration and print it")
    ap.add_argument("--pmc-summary", nargs=4, metavar=("FETCH", "WRITE", "COPY_FETCH", "COPY_WRITE"),
                    help="print the traffic summary of four rocprofv3 --pmc output directories and exit")
    ap.add_argument("--trace-summary", nargs=2, metavar=("DIR", "COMMAND"),
                    help="print the summary of a rocprofv3 --kernel-trace --stats directory and exit")
    ap.add_argument("--sq-summary", nargs=len(SQ_PASSES), metavar=tuple(f"SQ_{i}" for i in range(len(SQ_PASSES))),
                    help="print the SQ-counter summary of the rocprofv3 --pmc output directories of "
                         "sq_commands() and exit")
    args = ap.parse_args()
    if args.pmc_summary:
        print(pmc_summary(*args.pmc_summary, workload=args.workload))
        return
    if args.trace_summary:
        print(trace_summary(*args.trace_summary))
        return
    if args.sq_summary:
        print(sq_summary(args.sq_summary, workload=args.workload))
        return
    if args.gpus != 1:
        print(f"bench.py measures one GPU only (--gpus {args.gpus} requested); the op chain shards "
              f"per token with no communication, so N GPUs would run N independent copies.", file=sys.stderr)
        sys.exit(2)

    import torch

    import anelm

    if args.calibrate_copy:
        src = torch.randn(1 << 28, device="cuda")
        dst = torch.empty_like(src)
        ms = time_region(lambda: dst.copy_(src), 5)
        print(json.dumps(dict(calibration="device copy", bytes_read=1 << 30, bytes_written=1 << 30, ms=round(ms, 4),
                              GBps=round(2 * (1 << 30) / ms / 1e6, 1))))
        return

    anelm.lib()
    if args.only:
        if args.only in ATTN_WORKLOADS:
            r = measure_attention(anelm, ATTN_WORKLOADS[args.only], max(args.steps, 20))
        elif args.only in DN_WORKLOADS:
            r = measure_deltanet(anelm, DN_WORKLOADS[args.only], max(args.steps, 20))
        elif args.only == "sampling-64x151936":
            r = measure_sampler(anelm, max(args.steps, 20))
            r["frequency_penalty_0"] = measure_sampler(anelm, max(args.steps, 20), freq=0.0)
        elif args.only == "sampling-1x151936":
            r = measure_sampler(anelm, max(args.steps, 20), rows=1)
        elif args.only == "convert-qwen3-8b-bf16":
            r = measure_convert(anelm)
        elif args.only == "dropin-per-call":
            r = dropin_per_call()
        elif args.only in Q3_WORKLOADS:
            import tempfile

            with tempfile.TemporaryDirectory() as wd:
                src = os.path.join(wd, "qwen3-0.6b-shaped.safetensors")
                make_blob_checkpoint(src)
                r = measure_qwen3(anelm, src, Q3_WORKLOADS[args.only])
                if not args.no_cpu:
                    r["cpu"] = cpu_qwen3(src)
        elif args.only == "blobs-qwen3-0.6b":
            import tempfile

            with tempfile.TemporaryDirectory() as wd:
                src, r = measure_blobs(anelm, wd)
                if not args.no_cpu:
                    r["cpu"] = cpu_blobs(src, wd)
        else:
            r = measure_chain(WORKLOADS[args.only], args.steps, args.warmup, per_op=True)
        print(json.dumps({args.only: r}))
        return
    if args.workload not in WORKLOADS:
        raise SystemExit(f"--workload {args.workload}: an op-chain workload is needed here ({', '.join(WORKLOADS)})")
    w = WORKLOADS[args.workload]
    head = measure_chain(w, args.steps, args.warmup, per_op=not args.chain_only, chain_only=args.chain_only,
                         op_steps=args.steps)
    if args.chain_only:
        print(json.dumps({args.workload: head}))
        return
    # The headline step, op-major: each op over all layers as one graph, x,
    # xn and h rotating over the buffer sets, so no launch reads what the
    # launch before it wrote (each op's launches touch >= 256 MB, the
    # Infinity Cache's size, at the 8B prefill shape): the step time is the
    # sum of the five ops' times and every byte counted comes from HBM.  The
    # layer-major chain (the model's order) is reported beside it: there
    # each op reads what the op before it wrote, partly from that cache.
    env_ms = sum(head["ops"][n]["ms_all_layers"] for n in OPS)
    env = dict(ms_per_step=round(env_ms, 4), us_per_layer_chain=round(env_ms * 1e3 / w["layers"], 3),
               GBps=round(head["chain_bytes"] / env_ms / 1e6, 1),
               frac=round(head["chain_bytes"] / env_ms / 1e6 / HBM_PEAK_GBPS, 4),
               tokens_per_s=round(w["T"] / (env_ms / 1e3), 1))
    layer_major = {k: head[k] for k in ("ms_per_step", "us_per_layer_chain", "GBps", "frac", "tokens_per_s")}
    layer_major["note"] = ("the five ops layer by layer (models/llm/qwen3.cpp:502-528 order), one graph per step, "
                           "x/xn/h rotating over the buffer sets across layers; within a layer an op reads what the "
                           "launch before it wrote, partly from the 256 MB Infinity Cache, so this includes "
                           "within-layer Infinity-Cache reuse")
    ob = op_bytes(w)
    dom = max(OPS, key=lambda n: ob[n])
    roof = dict(bound="hbm", kernel=dom, achieved=head["ops"][dom]["GBps"], peak=HBM_PEAK_GBPS, unit="GB/s",
                frac=head["ops"][dom]["frac"], traffic=load_traffic(args.workload, dom),
                algorithmic_bytes_per_launch=ob[dom],
                traffic_source=f"profiles/pmc_traffic_{args.workload}.txt (FETCH_SIZE, WRITE_SIZE per dispatch, "
                               f"copy-calibrated)")
    configs = {}
    cpu_configs = {}
    if not args.headline_only:
        for name, wl in WORKLOADS.items():
            if name != args.workload:
                configs[name] = measure_chain(wl, max(args.steps, 20), args.warmup, per_op=False)
        configs["sampling-64x151936"] = measure_sampler(anelm, max(args.steps, 20))
        configs["sampling-64x151936"]["frequency_penalty_0"] = {
            k: v for k, v in measure_sampler(anelm, max(args.steps, 20), freq=0.0).items() if k != "note"}
        # one row: what the reference samples per decode step (generate.cpp:80-129)
        configs["sampling-1x151936"] = measure_sampler(anelm, max(args.steps, 20), rows=1)
        for name, aw in ATTN_WORKLOADS.items():
            configs[name] = measure_attention(anelm, aw, max(args.steps, 20))
        for name, dw in DN_WORKLOADS.items():
            configs[name] = measure_deltanet(anelm, dw, max(args.steps, 20))
        import tempfile

        with tempfile.TemporaryDirectory() as wd:
            src, configs["blobs-qwen3-0.6b"] = measure_blobs(anelm, wd)
            if not args.no_cpu:
                cpu_configs["blobs-qwen3-0.6b"] = cpu_blobs(src, wd)
            for name, qw in Q3_WORKLOADS.items():
                configs[name] = measure_qwen3(anelm, src, qw)
            if not args.no_cpu:
                cpu_configs["qwen3-0.6b-decode-step"] = cpu_qwen3(src)
        configs["convert-qwen3-8b-bf16"] = measure_convert(anelm)
    cpu = None
    if not args.no_cpu:
        cpu = cpu_chain(w, args.cpu_seconds)
        one = cpu_chain(w, max(2.0, args.cpu_seconds / 4), max_tokens=64, layers=2, threads=1)
        cpu["single_thread"] = {k: one[k] for k in ("value", "unit", "cores", "us_per_layer_chain", "sample")}
        if not args.headline_only:
            for name, wl in WORKLOADS.items():
                if name != args.workload:
                    cpu_configs[name] = cpu_chain(wl, 1.5, max_tokens=256, layers=2)
            cpu_configs["sampling-64x151936"] = cpu_sampler(1.5)
            cpu_configs["sampling-64x151936"]["frequency_penalty_0"] = {
                k: v for k, v in cpu_sampler(1.0, freq=0.0).items() if k in ("us", "GBps")}
            cpu_configs["sampling-1x151936"] = cpu_sampler(0.5, rows=1)
            cpu_configs["attention-qwen3-8b-decode"] = cpu_attention(ATTN_WORKLOADS["attention-qwen3-8b-decode-b1"], 1.5)
            cpu_configs["convert-qwen3-8b-bf16"] = cpu_convert(1.5)
    dropin = None
    if not args.no_cpu and not args.headline_only:
        dropin = dropin_per_call()
    out = {
        "metric": METRIC,
        "value": env["GBps"],
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": env["ms_per_step"],
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic: seeded device randn activations N(0,1), fp16 gammas 1+N(0,0.02), distinct inputs per "
                "layer; residual stream and outputs rotating over 4 buffer sets across layers",
        "config": dict(workload=args.workload, tokens=w["T"], hidden=w["H"], q_heads=w["nq"], kv_heads=w["nk"],
                       head_dim=D, intermediate=w["I"], layers=w["layers"], rope_theta=THETA,
                       positions=w["positions"],
                       launch="op-major step: one HIP graph per op over all layers, step time = sum of the five; "
                              "every byte from HBM"),
        "frac_of_hbm_peak": env["frac"],
        "us_per_layer_chain": env["us_per_layer_chain"],
        "tokens_per_s": env["tokens_per_s"],
        "chain_bytes_per_step": head["chain_bytes"],
        "buffer_sets": head["buffer_sets"],
        "layer_major_chain": layer_major,
        "carried_x": head.get("carried_x"),
        "one_launch_per_layer": head.get("one_launch_per_layer"),
        "roofline": roof,
        "cpu_baseline": cpu,
        "ops": head["ops"],
        "configs": configs,
        "cpu_configs": cpu_configs,
        "dropin_per_call": dropin,
    }
    print(json.dumps(out))


if __name__ == "__main__":
    main()
