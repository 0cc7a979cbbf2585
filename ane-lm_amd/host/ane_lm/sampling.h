// Drop-in declarations for the reference's core/sampling.h (Lolendorka/ANE-LM),
// backed by libanelm_hip.so.  Identical struct, defaults and signature
// (core/sampling.h:7-16).  sample_token draws r = (float)drand48() on the
// host exactly when the reference does (temperature > 0), so a caller's
// srand48 seed reproduces the reference's token stream.
#pragma once

#include <vector>

namespace ane_lm {

struct SamplingParams {
    float temperature = 0.6f;
    float repetition_penalty = 1.2f;
    int repetition_context_size = 256;
    float frequency_penalty = 0.1f;
};

int sample_token(const float* logits, int vocab_size,
                 const SamplingParams& params,
                 const std::vector<int>& recent_tokens = {});

}  // namespace ane_lm
