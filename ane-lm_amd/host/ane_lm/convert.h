// Drop-in for the reference's weight convert (include/ane_lm/common.h:81-83,
// bf16_to_f16_vec).  common.h defines it inline, so it cannot be replaced at
// link time; the hook is at its two call sites, core/safetensors.cpp:335
// (write_ane_blob) and core/ane_runtime.cpp:207 (build_weight_blob), which
// call ane_lm::hip::bf16_to_f16_vec instead.  Bit-exact with the reference's
// truncating convert.  Host pointers; synchronous.
#pragma once

#include <cstddef>
#include <cstdint>

namespace ane_lm {
namespace hip {
void bf16_to_f16_vec(uint16_t* out, const uint16_t* in, int n);
// size_t-count form for tensors of 2^31 elements or more
void bf16_to_f16_vec_n(uint16_t* out, const uint16_t* in, size_t n);
}  // namespace hip
}  // namespace ane_lm
