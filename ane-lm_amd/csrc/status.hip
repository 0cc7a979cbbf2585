// Per-thread error reporting, version, and the host-side inverse-frequency
// helper shared by the RoPE entry points.
#include <cmath>
#include <cstdarg>
#include <cstdio>
#include <mutex>

#include "anelm_common.hpp"

namespace anelm {

static thread_local char t_last_error[512] = {0};

int fail(int code, const char* fmt, ...) {
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(t_last_error, sizeof(t_last_error), fmt, ap);
    va_end(ap);
    return code;
}

void clear_error() { t_last_error[0] = 0; }

int launch_status(const char* what) {
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return fail(ANELM_ERR_HIP, "%s: launch failed: %s", what, hipGetErrorString(e));
    return ANELM_OK;
}

// The 64..512 powf evaluations are cached per thread for the last
// (rot_dim, theta) pair, so repeated launches do not re-evaluate them.
void rope_inv_freq(InvFreq* out, int rot_dim, float theta) {
    static thread_local InvFreq cache;
    static thread_local int cache_rot = -1;
    static thread_local float cache_theta = 0.0f;
    if (cache_rot != rot_dim || !(cache_theta == theta)) {
        for (int j = 0, i = 0; i < rot_dim; i += 2, j++)
            cache.v[j] = 1.0f / powf(theta, (float)i / (float)rot_dim);
        cache_rot = rot_dim;
        cache_theta = theta;
    }
    *out = cache;
}

}  // namespace anelm

extern "C" const char* anelm_last_error(void) { return anelm::t_last_error; }

extern "C" int anelm_version(void) { return 100; }
