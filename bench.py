"""Benchmark of the fused layer-op chain on one MI355X.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--workload NAME]

A step is one pass of the op chain over all layers of the workload:
  (1) RMSNorm  (2) q/k-norm + RoPE  (3) residual add + RMSNorm
  (4) SwiGLU   (5) residual add
(models/llm/qwen3.cpp:502-528), on synthetic device-resident inputs with
distinct per-layer inputs.  `value` is the chain's algorithmic HBM bytes per
step divided by the measured step time (GB/s).  Prints one JSON line.
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

WORKLOADS = {
    # Qwen3-8B-shaped prefill, T=8192 (the target configuration)
    "qwen3-8b-prefill": dict(T=8192, H=4096, nq=32, nk=8, I=12288, layers=36, positions="sequential", pmax=8192,
                             convert=True),
    # Qwen3-0.6B prefill, T=2048
    "qwen3-0.6b-prefill": dict(T=2048, H=1024, nq=16, nk=8, I=3072, layers=28, positions="sequential", pmax=2048,
                               convert=False),
    # Qwen3-4B batched decode, 64 sequences
    "qwen3-4b-decode-b64": dict(T=64, H=2560, nq=32, nk=8, I=9728, layers=36, positions="uniform", pmax=32768,
                                convert=False),
    # Qwen3-0.6B single-token decode
    "qwen3-0.6b-decode": dict(T=1, H=1024, nq=16, nk=8, I=3072, layers=28, positions="uniform", pmax=4096,
                              convert=False),
}

OPS = ["rmsnorm", "qknorm_rope", "add_rmsnorm", "silu_mul", "residual_add"]


def op_bytes(w):
    """Algorithmic (compulsory) HBM bytes per launch of each op: every input
    read once, every output written once (fp32 activations; gammas ignored)."""
    T, H, I, nh = w["T"], w["H"], w["I"], w["nq"] + w["nk"]
    return {
        "rmsnorm": 2 * T * H * 4,                        # read x, write xn
        "qknorm_rope": 2 * T * nh * D * 4 + T * (D // 2) * 2 * 4,  # q,k in place + cos/sin rows
        "add_rmsnorm": 4 * T * H * 4,                    # read x, y; write x, xn
        "silu_mul": 3 * T * I * 4,                       # read g, u; write h
        "residual_add": 3 * T * H * 4,                   # read x, y; write x
    }


def qwen3_8b_tensor_sizes():
    H, I, V, L = 4096, 12288, 151936, 36
    sizes = [V * H, V * H, H]
    for _ in range(L):
        sizes += [H * H, 1024 * H, 1024 * H, H * H, I * H, I * H, H * I, H, H, D, D]
    return sizes


class Chain:
    def __init__(self, w, seed=0):
        import torch

        import anelm

        self.w, self.hip = w, anelm
        T, H, I, nq, nk, L = w["T"], w["H"], w["I"], w["nq"], w["nk"], w["layers"]
        g = torch.Generator(device="cuda").manual_seed(seed)
        rn = lambda *s: torch.randn(*s, generator=g, device="cuda", dtype=torch.float32)
        gamma = lambda n: (1.0 + 0.02 * rn(n)).to(torch.float16)
        self.x = rn(T, H)
        self.xn = torch.empty(T, H, device="cuda")
        self.h = torch.empty(T, I, device="cuda")
        self.layers = []
        for _ in range(L):
            self.layers.append(dict(attn=rn(T, H), mlp=rn(T, H), q=rn(T, nq * D), k=rn(T, nk * D), g=rn(T, I),
                                    u=rn(T, I), w_in=gamma(H), w_post=gamma(H), wq=gamma(D), wk=gamma(D)))
        if w["positions"] == "sequential":
            self.pos = torch.arange(T, device="cuda", dtype=torch.int32)
        else:
            self.pos = torch.randint(0, w["pmax"], (T,), generator=g, device="cuda", dtype=torch.int32)
        self.cos = torch.empty(16384, D // 2, device="cuda")
        self.sin = torch.empty(16384, D // 2, device="cuda")
        anelm.rope_table(self.cos, self.sin, THETA)

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

    def step(self):
        for Ld in self.layers:
            for name in OPS:
                self.op(name, Ld)


def time_region(fn, reps):
    import torch

    s, e = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    s.record()
    for _ in range(reps):
        fn()
    e.record()
    torch.cuda.synchronize()
    return s.elapsed_time(e) / reps  # ms


def bench_convert(hip, reps=3):
    """bf16->fp16 of the 8,190,735,360-parameter Qwen3-8B set, one call per tensor."""
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
    views = []
    off = 0
    for m in sizes:
        views.append((dst[off:off + m], src[off:off + m]))
        off += m

    def run():
        for d, s in views:
            hip.bf16_to_f16(d, s)

    run()
    ms = time_region(run, reps)
    del src, dst, views
    torch.cuda.empty_cache()
    byt = 4 * n
    return dict(params=n, ms=round(ms, 4), GBps=round(byt / ms / 1e6, 1), frac=round(byt / ms / 1e6 / HBM_PEAK_GBPS, 4),
                bytes=byt, launches=len(sizes))


def cpu_baseline(w, target_s):
    """The oracle's per-token layer chain on the host's cores over a bounded
    sample of the workload: T_s tokens x 4 layers with distinct inputs,
    repeated until ~target_s seconds have elapsed."""
    import numpy as np

    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import oracle

    T = min(w["T"], 512)
    H, I, nq, nk = w["H"], w["I"], w["nq"], w["nk"]
    Ls = 4
    rng = np.random.default_rng(5)
    rn = lambda *s: rng.standard_normal(s, dtype=np.float32)
    lay = [dict(attn=rn(T, H), mlp=rn(T, H), q=rn(T, nq * D), k=rn(T, nk * D), g=rn(T, I), u=rn(T, I)) for _ in range(Ls)]
    gam = lambda n: (1 + 0.02 * rng.standard_normal(n)).astype(np.float16).astype(np.float32)
    w_in, w_post, wq, wk = gam(H), gam(H), gam(D), gam(D)
    x, xn, h = rn(T, H), np.empty((T, H), np.float32), np.empty((T, I), np.float32)
    pos = (np.arange(T) % w["pmax"]).astype(np.int32)
    c, s = oracle.rope_table(16384, D, THETA)
    threads = oracle.max_threads()
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
    gbps = per_layer_bytes * Ls * passes / el / 1e9
    return dict(value=round(gbps, 2), unit="GB/s", cores=threads, kind="port",
                sample=f"oracle layer chain (per-token loop as the reference), {T} tokens x {Ls} distinct layers "
                       f"of the workload's shapes, {passes} passes in {el:.1f} s on {threads} OpenMP threads",
                us_per_layer_chain_full_T=round(el / (Ls * passes) * (w["T"] / T) * 1e6, 1))


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--workload", default="qwen3-8b-prefill", choices=sorted(WORKLOADS))
    ap.add_argument("--cpu-seconds", type=float, default=8.0)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--no-convert", action="store_true")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py: this build measures one GPU only (--gpus {args.gpus} requested); the op chain shards "
              f"per token with no communication, so N GPUs would run N independent copies.", file=sys.stderr)
        sys.exit(2)

    import torch

    import anelm

    anelm.lib()
    w = WORKLOADS[args.workload]
    chain = Chain(w)
    for _ in range(args.warmup):
        chain.step()
    ms = time_region(chain.step, args.steps)

    # per-op launch durations over the same per-layer buffers
    ob = op_bytes(w)
    ops = {}
    reps = 3 if w["T"] >= 1024 else 50
    for name in OPS:
        t = time_region(lambda: [chain.op(name, Ld) for Ld in chain.layers], reps) / len(chain.layers)
        ops[name] = dict(us=round(t * 1e3, 2), GBps=round(ob[name] / t / 1e6, 1),
                         frac=round(ob[name] / t / 1e6 / HBM_PEAK_GBPS, 4), bytes=ob[name])
    layer_bytes = sum(ob.values())
    chain_bytes = layer_bytes * w["layers"]
    gbps = chain_bytes / ms / 1e6
    dom = max(OPS, key=lambda n: ob[n])
    roof = dict(bound="hbm", kernel=dom, achieved=ops[dom]["GBps"], peak=HBM_PEAK_GBPS, unit="GB/s",
                frac=ops[dom]["frac"], traffic=None, algorithmic_bytes_per_launch=ob[dom])
    del chain
    torch.cuda.empty_cache()

    extras = {}
    if w["convert"] and not args.no_convert:
        extras["convert_bf16_to_f16"] = bench_convert(anelm)
    cpu = None if args.no_cpu else cpu_baseline(w, args.cpu_seconds)
    out = {
        "metric": METRIC,
        "value": round(gbps, 1),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic: seeded device randn activations N(0,1), fp16 gammas 1+N(0,0.02), distinct inputs per layer",
        "config": dict(workload=args.workload, tokens=w["T"], hidden=w["H"], q_heads=w["nq"], kv_heads=w["nk"],
                       head_dim=D, intermediate=w["I"], layers=w["layers"], rope_theta=THETA,
                       positions=w["positions"]),
        "frac_of_hbm_peak": round(gbps / HBM_PEAK_GBPS, 4),
        "us_per_layer_chain": round(ms * 1e3 / w["layers"], 2),
        "tokens_per_s": round(w["T"] / (ms / 1e3), 1),
        "chain_bytes_per_step": chain_bytes,
        "roofline": roof,
        "cpu_baseline": cpu,
        "ops": ops,
        **extras,
    }
    print(json.dumps(out))


if __name__ == "__main__":
    main()
