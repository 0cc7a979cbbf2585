// Per-call wall time of the ane_lm:: drop-in functions, called as the
// reference's unchanged callers call them (host pointers in and out, one
// synchronous call per op), beside the oracle's single-thread CPU
// restatement of the same function on the same inputs:
//   rmsnorm at dim 1024      -- the per-token norms, models/llm/qwen3.cpp:503, :516
//   rmsnorm at dim 128 x 40  -- the per-head q/k norms of one layer from 8
//                               threads at once, models/llm/qwen3.cpp:451-461
//   sample_token at 151936   -- once per generated token, generate.cpp:80, :129
// and the additive entries for the ops the reference performs inline, at the
// Qwen3-8B per-token shapes, each beside the oracle's same function on one
// thread:
//   hip::qknorm_rope_qwen3, 32 q + 8 k heads -- a layer's 40 head norms and
//                               RoPE in one call, models/llm/qwen3.cpp:444-472
//   hip::residual_add at 4096 -- models/llm/qwen3.cpp:516, :527
//   hip::silu_mul at 12288    -- the fused_ffn activation, core/ane_runtime.cpp:393-395
// Prints one JSON line (microseconds per call: mean and median over the
// timed calls).  Needs a GPU.
#include <algorithm>
#include <atomic>
#include <chrono>
#include <cstdio>
#include <cstdlib>
#include <random>
#include <thread>
#include <vector>

#include "anelm_oracle.h"
#include "ane_lm/cpu_ops.h"
#include "ane_lm/sampling.h"

namespace {

using Clock = std::chrono::steady_clock;

struct Stat {
    double mean_us, median_us;
    int calls;
};

// Times fn() `calls` times after `warmup` untimed calls.
template <class F>
Stat time_calls(F&& fn, int warmup, int calls) {
    for (int i = 0; i < warmup; i++) fn();
    std::vector<double> t(calls);
    for (int i = 0; i < calls; i++) {
        auto a = Clock::now();
        fn();
        t[i] = std::chrono::duration<double, std::micro>(Clock::now() - a).count();
    }
    double sum = 0;
    for (double v : t) sum += v;
    std::nth_element(t.begin(), t.begin() + calls / 2, t.end());
    return {sum / calls, t[calls / 2], calls};
}

void put(const char* key, const Stat& dropin, const Stat& cpu, bool last) {
    printf("\"%s\": {\"dropin_us\": %.2f, \"dropin_median_us\": %.2f, \"dropin_calls\": %d, "
           "\"oracle_cpu_us\": %.2f, \"oracle_cpu_median_us\": %.2f, \"oracle_calls\": %d, "
           "\"dropin_over_cpu\": %.3f}%s",
           key, dropin.mean_us, dropin.median_us, dropin.calls, cpu.mean_us, cpu.median_us, cpu.calls,
           dropin.mean_us / cpu.mean_us, last ? "" : ", ");
}

}  // namespace

int main() {
    std::mt19937 gen(7);
    std::normal_distribution<float> nd(0.f, 1.f);
    auto randv = [&](size_t n, float scale = 1.f) {
        std::vector<float> v(n);
        for (auto& x : v) x = nd(gen) * scale;
        return v;
    };
    printf("{");

    for (int dim : {1024, 128}) {
        auto x = randv(dim), w = randv(dim, 0.02f);
        for (auto& e : w) e += 1.f;
        std::vector<float> out(dim);
        Stat g = time_calls([&] { ane_lm::rmsnorm(out.data(), x.data(), w.data(), dim, 1e-6f); }, 50, 2000);
        Stat c = time_calls([&] { orc_rmsnorm(out.data(), x.data(), w.data(), dim, 1e-6f); }, 200, 20000);
        char key[32];
        snprintf(key, sizeof key, "rmsnorm_%d", dim);
        put(key, g, c, false);
    }

    // one layer's 32 q-head and 8 k-head norms on 8 persistent worker threads
    // (GCD's dispatch_apply reuses its pool's threads), 5 heads each, each
    // rmsnorm call in place on its own head (qwen3.cpp:451-461)
    {
        const int heads = 40, hd = 128, nthreads = 8;
        auto qk = randv((size_t)heads * hd), w = randv(hd, 0.02f);
        for (auto& e : w) e += 1.f;
        std::atomic<int> gen_no{0}, done{0}, use_gpu{0};
        std::atomic<bool> stop{false};
        std::vector<std::thread> pool;
        for (int t = 0; t < nthreads; t++)
            pool.emplace_back([&, t] {
                int seen = 0;
                for (;;) {
                    int g;
                    while ((g = gen_no.load(std::memory_order_acquire)) == seen && !stop.load()) std::this_thread::yield();
                    if (stop.load()) return;
                    seen = g;
                    for (int h = t; h < heads; h += nthreads) {
                        float* p = &qk[(size_t)h * hd];
                        if (use_gpu.load())
                            ane_lm::rmsnorm(p, p, w.data(), hd, 1e-6f);
                        else
                            orc_rmsnorm(p, p, w.data(), hd, 1e-6f);
                    }
                    done.fetch_add(1, std::memory_order_release);
                }
            });
        auto layer = [&](bool gpu) {
            use_gpu.store(gpu ? 1 : 0);
            done.store(0);
            gen_no.fetch_add(1, std::memory_order_release);
            while (done.load(std::memory_order_acquire) < nthreads) std::this_thread::yield();
        };
        Stat g = time_calls([&] { layer(true); }, 10, 300);
        Stat c = time_calls([&] { layer(false); }, 10, 300);
        stop.store(true);
        for (auto& th : pool) th.join();
        put("rmsnorm_128_x40_heads_8_threads_per_layer", g, c, false);
    }

    // one token's 40 head norms + RoPE in one call (table row of position 1234)
    {
        const int nq = 32, nk = 8, hd = 128;
        auto q = randv((size_t)nq * hd), k = randv((size_t)nk * hd), wq = randv(hd, 0.02f), wk = randv(hd, 0.02f);
        for (auto& e : wq) e += 1.f;
        for (auto& e : wk) e += 1.f;
        std::vector<float> ctab((size_t)2048 * hd / 2), stab(ctab.size());
        orc_rope_table(ctab.data(), stab.data(), 2048, hd, 1e6f);
        const float* cr = &ctab[(size_t)1234 * hd / 2];
        const float* sr = &stab[(size_t)1234 * hd / 2];
        Stat g = time_calls([&] { ane_lm::hip::qknorm_rope_qwen3(q.data(), k.data(), nq, nk, hd, wq.data(), wk.data(),
                                                                 1e-6f, 1234, 1e6f, cr, sr); }, 50, 2000);
        const int32_t pos = 0;   // the row as a one-row table
        Stat c = time_calls([&] { orc_qknorm_rope(q.data(), k.data(), (long)nq * hd, (long)nk * hd, wq.data(), wk.data(),
                                                  &pos, cr, sr, 1, 1e6f, 1, nq, nk, hd, 1e-6f, 1); }, 200, 20000);
        put("hip_qknorm_rope_qwen3_32q_8k", g, c, false);
    }
    {
        const int n = 4096;
        auto x = randv(n), y = randv(n);
        Stat g = time_calls([&] { ane_lm::hip::residual_add(x.data(), y.data(), n); }, 50, 2000);
        Stat c = time_calls([&] { orc_residual_add(x.data(), y.data(), (size_t)n, 1); }, 200, 20000);
        put("hip_residual_add_4096", g, c, false);
    }
    {
        const int n = 12288;
        auto gt = randv(n), ut = randv(n);
        std::vector<float> h(n);
        Stat g = time_calls([&] { ane_lm::hip::silu_mul(h.data(), gt.data(), ut.data(), n); }, 50, 2000);
        Stat c = time_calls([&] { orc_silu_mul(h.data(), gt.data(), ut.data(), (size_t)n, 1); }, 200, 20000);
        put("hip_silu_mul_12288", g, c, false);
    }

    {
        const int V = 151936;
        auto logits = randv(V, 3.f);
        std::vector<int> recent(256);
        for (int i = 0; i < 256; i++) recent[i] = (int)(gen() % V);
        ane_lm::SamplingParams p;   // temperature 0.6, repetition 1.2 over 256, frequency 0.1
        srand48(1);
        Stat g = time_calls([&] { (void)ane_lm::sample_token(logits.data(), V, p, recent); }, 10, 200);
        Stat c = time_calls(
            [&] {
                (void)orc_sample_token(logits.data(), V, p.temperature, p.repetition_penalty,
                                       p.repetition_context_size, p.frequency_penalty, recent.data(),
                                       (int)recent.size(), 0.37f, nullptr);
            },
            3, 60);
        put("sample_token_151936", g, c, true);
    }
    printf("}\n");
    return 0;
}
