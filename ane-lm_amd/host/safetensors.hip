// Safetensors reader with device upload, and the ANE weight-blob writer with
// the bf16 -> fp16 convert on the GPU.  Replaces core/safetensors.cpp:
//   :58-245   header parse and mmap (SafeTensors::open / parse_header)
//   :266-313  the loaders (load_bf16_to_f32, load_f32_direct, get_bf16_ptr)
//   :316-383  write_ane_blob / write_ane_blobs (the `convert` command)
// for a device-resident runtime: tensors go from the page cache through
// pinned staging to HBM, and blobs come back converted, with the host
// copies, DMA and kernels of consecutive chunks overlapped.
#include <hip/hip_runtime.h>

#include <fcntl.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <cerrno>
#include <cstdio>
#include <cstring>
#include <string>
#include <vector>

#include "anelm_common.hpp"

using anelm::fail;
using anelm::clear_error;

namespace {

constexpr size_t kChunkBytes = (size_t)32 << 20;   // staging per pipeline slot

struct StTensor {
    std::string name;   // the raw text between the key's quotes, as the reference keeps it
    int dtype;
    int ndims;
    int64_t shape[8];
    int64_t numel;
    uint64_t offset;    // into the data block
    uint64_t nbytes;
};

int dtype_code(const std::string& s) {
    if (s == "BF16") return ANELM_BF16;
    if (s == "F16") return ANELM_F16;
    if (s == "F32") return ANELM_F32;
    if (s == "F64") return ANELM_ST_F64;
    if (s == "I32") return ANELM_ST_I32;
    if (s == "I64") return ANELM_ST_I64;
    if (s == "U8") return ANELM_ST_U8;
    return ANELM_ST_UNKNOWN;
}

int dtype_size(int d) {
    switch (d) {
        case ANELM_BF16: case ANELM_F16: return 2;
        case ANELM_F32: case ANELM_ST_I32: return 4;
        case ANELM_ST_F64: case ANELM_ST_I64: return 8;
        case ANELM_ST_U8: return 1;
        default: return 0;
    }
}

// Minimal JSON reader for the safetensors header: an object whose values are
// objects {"dtype": str, "shape": [int...], "data_offsets": [int, int]},
// plus an optional "__metadata__" object that is skipped.
struct Json {
    const char* s;
    size_t n, i = 0;
    void ws() {
        while (i < n && (s[i] == ' ' || s[i] == '\n' || s[i] == '\r' || s[i] == '\t')) i++;
    }
    bool eat(char c) {
        ws();
        if (i < n && s[i] == c) {
            i++;
            return true;
        }
        return false;
    }
    bool peek(char c) {
        ws();
        return i < n && s[i] == c;
    }
    bool str(std::string& out) {
        ws();
        if (i >= n || s[i] != '"') return false;
        const size_t st = ++i;
        while (i < n && s[i] != '"') i += s[i] == '\\' ? 2 : 1;
        if (i >= n) return false;
        out.assign(s + st, i - st);
        i++;
        return true;
    }
    bool integer(int64_t& v) {
        ws();
        bool neg = false;
        if (i < n && s[i] == '-') {
            neg = true;
            i++;
        }
        if (i >= n || s[i] < '0' || s[i] > '9') return false;
        uint64_t x = 0;
        while (i < n && s[i] >= '0' && s[i] <= '9') {
            if (x > (UINT64_MAX - 9) / 10) return false;
            x = x * 10 + (uint64_t)(s[i++] - '0');
        }
        if (x > (uint64_t)INT64_MAX) return false;
        v = neg ? -(int64_t)x : (int64_t)x;
        return true;
    }
    bool skip(int depth = 0) {
        ws();
        if (i >= n || depth > 64) return false;
        if (s[i] == '"') {
            std::string t;
            return str(t);
        }
        if (s[i] == '{' || s[i] == '[') {
            const char close = s[i] == '{' ? '}' : ']';
            const bool obj = s[i] == '{';
            i++;
            if (eat(close)) return true;
            do {
                if (obj) {
                    std::string k;
                    if (!str(k) || !eat(':')) return false;
                }
                if (!skip(depth + 1)) return false;
            } while (eat(','));
            return eat(close);
        }
        while (i < n && s[i] != ',' && s[i] != '}' && s[i] != ']' && s[i] != ' ' && s[i] != '\n') i++;
        return true;
    }
};

bool parse_tensor(Json& j, StTensor& t) {
    if (!j.eat('{')) return false;
    bool have_dt = false, have_shape = false, have_off = false;
    int64_t a = 0, b = 0;
    if (!j.peek('}')) {
        do {
            std::string k;
            if (!j.str(k) || !j.eat(':')) return false;
            if (k == "dtype") {
                std::string d;
                if (!j.str(d)) return false;
                t.dtype = dtype_code(d);
                have_dt = true;
            } else if (k == "shape") {
                if (!j.eat('[')) return false;
                t.ndims = 0;
                if (!j.eat(']')) {
                    do {
                        int64_t v;
                        if (!j.integer(v) || v < 0 || t.ndims >= 8) return false;
                        t.shape[t.ndims++] = v;
                    } while (j.eat(','));
                    if (!j.eat(']')) return false;
                }
                have_shape = true;
            } else if (k == "data_offsets") {
                if (!j.eat('[') || !j.integer(a) || !j.eat(',') || !j.integer(b) || !j.eat(']')) return false;
                have_off = true;
            } else if (!j.skip()) {
                return false;
            }
        } while (j.eat(','));
    }
    if (!j.eat('}') || !have_dt || !have_shape || !have_off || a < 0 || b < a) return false;
    t.offset = (uint64_t)a;
    t.nbytes = (uint64_t)(b - a);
    t.numel = 1;
    for (int d = 0; d < t.ndims; d++) {
        if (t.shape[d] && t.numel > INT64_MAX / t.shape[d]) return false;
        t.numel *= t.shape[d];
    }
    return true;
}

int hip_fail(hipError_t e, const char* what) {
    return fail(ANELM_ERR_HIP, "%s: %s", what, hipGetErrorString(e));
}

// mkdir -p of the directory part of path
bool make_parents(const std::string& path) {
    for (size_t p = path.find('/', 1); p != std::string::npos; p = path.find('/', p + 1)) {
        const std::string d = path.substr(0, p);
        if (mkdir(d.c_str(), 0755) != 0 && errno != EEXIST) return false;
    }
    return true;
}

// Pinned host and device staging for a two-slot pipeline.  Every use of a
// slot ends with its event recorded; wait() blocks until the slot's last use
// is complete (a slot never used is free).
struct Pipeline {
    char* hin[2] = {nullptr, nullptr};
    char* hout[2] = {nullptr, nullptr};
    char* dev[2] = {nullptr, nullptr};
    hipEvent_t ev[2] = {nullptr, nullptr};
    bool recorded[2] = {false, false};
    int init(bool with_out) {
        hipError_t e;
        for (int k = 0; k < 2; k++) {
            if ((e = hipHostMalloc(reinterpret_cast<void**>(&hin[k]), kChunkBytes, hipHostMallocDefault)) != hipSuccess)
                return hip_fail(e, "hipHostMalloc");
            if (with_out &&
                (e = hipHostMalloc(reinterpret_cast<void**>(&hout[k]), kChunkBytes, hipHostMallocDefault)) != hipSuccess)
                return hip_fail(e, "hipHostMalloc");
            if ((e = hipMalloc(reinterpret_cast<void**>(&dev[k]), kChunkBytes)) != hipSuccess) return hip_fail(e, "hipMalloc");
            if ((e = hipEventCreateWithFlags(&ev[k], hipEventDisableTiming)) != hipSuccess) return hip_fail(e, "hipEventCreate");
        }
        return ANELM_OK;
    }
    hipError_t wait(int k) { return recorded[k] ? hipEventSynchronize(ev[k]) : hipSuccess; }
    hipError_t record(int k, hipStream_t st) {
        const hipError_t e = hipEventRecord(ev[k], st);
        recorded[k] = e == hipSuccess;
        return e;
    }
    // teardown: a failure here has nowhere to go (the call that owns the
    // pipeline has already returned its status), so results are dropped
    ~Pipeline() {
        for (int k = 0; k < 2; k++) {
            if (ev[k]) {
                (void)wait(k);
                (void)hipEventDestroy(ev[k]);
            }
            if (hin[k]) (void)hipHostFree(hin[k]);
            if (hout[k]) (void)hipHostFree(hout[k]);
            if (dev[k]) (void)hipFree(dev[k]);
        }
    }
};

}  // namespace

struct anelm_st {
    int fd = -1;
    void* base = nullptr;
    size_t size = 0;
    const uint8_t* data = nullptr;
    uint64_t data_size = 0;
    std::vector<StTensor> t;
    Pipeline* pipe = nullptr;   // staging for anelm_st_load, made on first use
    ~anelm_st() {
        delete pipe;
        if (base) munmap(base, size);
        if (fd >= 0) close(fd);
    }
};

extern "C" anelm_st* anelm_st_open(const char* path) {
    clear_error();
    if (!path) {
        fail(ANELM_ERR_INVALID, "st_open: null path");
        return nullptr;
    }
    anelm_st* h = new anelm_st();
    h->fd = open(path, O_RDONLY);
    struct stat sb;
    if (h->fd < 0 || fstat(h->fd, &sb) != 0) {
        fail(ANELM_ERR_INVALID, "st_open: cannot open %s: %s", path, strerror(errno));
        delete h;
        return nullptr;
    }
    h->size = (size_t)sb.st_size;
    if (h->size < 8) {
        fail(ANELM_ERR_INVALID, "st_open: %s is too short", path);
        delete h;
        return nullptr;
    }
    void* base = mmap(nullptr, h->size, PROT_READ, MAP_PRIVATE, h->fd, 0);
    if (base == MAP_FAILED) {
        fail(ANELM_ERR_INVALID, "st_open: mmap failed: %s", strerror(errno));
        delete h;
        return nullptr;
    }
    h->base = base;
    uint64_t hlen;
    memcpy(&hlen, base, 8);
    if (hlen > h->size - 8) {
        fail(ANELM_ERR_INVALID, "st_open: header length %llu beyond the file", (unsigned long long)hlen);
        delete h;
        return nullptr;
    }
    h->data = static_cast<const uint8_t*>(base) + 8 + hlen;
    h->data_size = h->size - 8 - hlen;
    Json j{static_cast<const char*>(base) + 8, (size_t)hlen};
    bool ok = j.eat('{');
    if (ok && !j.peek('}')) {
        do {
            std::string key;
            if (!j.str(key) || !j.eat(':')) {
                ok = false;
                break;
            }
            if (key == "__metadata__") {
                if (!j.skip()) ok = false;
                continue;
            }
            StTensor t{};
            t.name = key;
            if (!parse_tensor(j, t)) {
                ok = false;
                break;
            }
            const int es = dtype_size(t.dtype);
            // (numel * es could wrap; offset + nbytes = the end offset <= INT64_MAX cannot)
            const bool size_ok =
                !es || (t.nbytes % (uint64_t)es == 0 && (uint64_t)t.numel == t.nbytes / (uint64_t)es);
            if (t.offset + t.nbytes > h->data_size || !size_ok) {
                fail(ANELM_ERR_INVALID, "st_open: tensor %s: data_offsets and shape disagree or leave the file",
                     t.name.c_str());
                delete h;
                return nullptr;
            }
            h->t.push_back(t);
        } while (j.eat(','));
    }
    if (!ok || !j.eat('}')) {
        fail(ANELM_ERR_INVALID, "st_open: malformed header in %s", path);
        delete h;
        return nullptr;
    }
    return h;
}

extern "C" void anelm_st_close(anelm_st* h) { delete h; }

extern "C" long anelm_st_count(const anelm_st* h) { return h ? (long)h->t.size() : 0; }

extern "C" long anelm_st_find(const anelm_st* h, const char* name) {
    if (!h || !name) return -1;
    for (size_t i = 0; i < h->t.size(); i++)
        if (h->t[i].name == name) return (long)i;
    return -1;
}

extern "C" int anelm_st_info(const anelm_st* h, long i, const char** name, int* dtype, int* ndims, int64_t* shape,
                             uint64_t* offset, uint64_t* nbytes) {
    clear_error();
    if (!h || i < 0 || i >= (long)h->t.size()) return fail(ANELM_ERR_RANGE, "st_info: no tensor %ld", i);
    const StTensor& t = h->t[i];
    if (name) *name = t.name.c_str();
    if (dtype) *dtype = t.dtype;
    if (ndims) *ndims = t.ndims;
    if (shape)
        for (int d = 0; d < t.ndims; d++) shape[d] = t.shape[d];
    if (offset) *offset = t.offset;
    if (nbytes) *nbytes = t.nbytes;
    return ANELM_OK;
}

extern "C" const void* anelm_st_host_data(const anelm_st* h, long i) {
    if (!h || i < 0 || i >= (long)h->t.size()) return nullptr;
    return h->data + h->t[i].offset;
}

namespace {

// Staged upload of tensor t (already validated) to dst: a copy, or for a BF16
// tensor the widening to fp32 (plus 1.0f when plus1) or the fp16 convert.
int load_tensor(const anelm_st* h, const StTensor& t, void* dst, bool widen, bool plus1, bool to_f16, void* stream) {
    if (t.nbytes == 0) return ANELM_OK;
    hipStream_t st = anelm::as_stream(stream);
    anelm_st* hm = const_cast<anelm_st*>(h);
    if (!hm->pipe) {
        hm->pipe = new Pipeline();
        const int r0 = hm->pipe->init(false);
        if (r0) {
            delete hm->pipe;
            hm->pipe = nullptr;
            return r0;
        }
    }
    Pipeline& p = *hm->pipe;
    int rc = ANELM_OK;
    const uint8_t* src = h->data + t.offset;
    hipError_t e;
    for (uint64_t off = 0, c = 0; off < t.nbytes; off += kChunkBytes, c++) {
        const int k = (int)(c & 1);
        const size_t n = (size_t)(t.nbytes - off < kChunkBytes ? t.nbytes - off : kChunkBytes);
        // the slot's previous H2D (this call's chunk c-2, or a previous call's) is done
        if ((e = p.wait(k)) != hipSuccess) return hip_fail(e, "st_load");
        memcpy(p.hin[k], src + off, n);
        if (widen) {   // staged bf16 chunk, widened into place
            if ((e = hipMemcpyAsync(p.dev[k], p.hin[k], n, hipMemcpyHostToDevice, st)) != hipSuccess)
                return hip_fail(e, "st_load H2D");
            float* d = static_cast<float*>(dst) + off / 2;
            const uint16_t* s16 = reinterpret_cast<const uint16_t*>(p.dev[k]);
            rc = plus1 ? anelm_bf16_to_f32_plus1(d, s16, n / 2, stream) : anelm_bf16_to_f32(d, s16, n / 2, stream);
        } else {
            char* d = static_cast<char*>(dst) + off;
            if ((e = hipMemcpyAsync(d, p.hin[k], n, hipMemcpyHostToDevice, st)) != hipSuccess)
                return hip_fail(e, "st_load H2D");
            rc = to_f16 ? anelm_bf16_to_f16(reinterpret_cast<uint16_t*>(d), reinterpret_cast<const uint16_t*>(d), n / 2,
                                            stream)
                        : ANELM_OK;
        }
        if (rc) return rc;
        if ((e = p.record(k, st)) != hipSuccess) return hip_fail(e, "st_load");
    }
    if ((e = hipStreamSynchronize(st)) != hipSuccess) return hip_fail(e, "st_load");
    return ANELM_OK;
}

}  // namespace

// Tensor i to device memory dst as dst_dtype: the tensor's own dtype (a
// copy), or for a BF16 tensor ANELM_F32 (exact widening, the reference's
// load_bf16_to_f32) or ANELM_F16 (the truncating convert of the blobs).
extern "C" int anelm_st_load(const anelm_st* h, long i, void* dst, int dst_dtype, void* stream) {
    clear_error();
    if (!h || i < 0 || i >= (long)h->t.size()) return fail(ANELM_ERR_RANGE, "st_load: no tensor %ld", i);
    if (!dst) return fail(ANELM_ERR_INVALID, "st_load: null destination");
    const StTensor& t = h->t[i];
    const bool widen = t.dtype == ANELM_BF16 && dst_dtype == ANELM_F32;
    const bool to_f16 = t.dtype == ANELM_BF16 && dst_dtype == ANELM_F16;
    if (!widen && !to_f16 && dst_dtype != t.dtype)
        return fail(ANELM_ERR_INVALID, "st_load: %s cannot be loaded as dtype %d", t.name.c_str(), dst_dtype);
    return load_tensor(h, t, dst, widen, false, to_f16, stream);
}

// core/safetensors.cpp:299-306 (load_norm_weight): the widened BF16 weight
// plus 1.0f.  The reference adds the offset for i < expected_numel, so a
// non-positive count (no shape check there either) gives the plain widening.
extern "C" int anelm_st_load_norm(const anelm_st* h, long i, float* dst, long expected_numel, void* stream) {
    clear_error();
    if (!h || i < 0 || i >= (long)h->t.size()) return fail(ANELM_ERR_RANGE, "st_load_norm: no tensor %ld", i);
    if (!dst) return fail(ANELM_ERR_INVALID, "st_load_norm: null destination");
    const StTensor& t = h->t[i];
    if (t.dtype != ANELM_BF16) return fail(ANELM_ERR_INVALID, "st_load_norm: %s is not BF16", t.name.c_str());
    if (expected_numel > 0 && t.numel != expected_numel)
        return fail(ANELM_ERR_INVALID, "st_load_norm: shape mismatch for %s: expected %ld, got %lld", t.name.c_str(),
                    expected_numel, (long long)t.numel);
    return load_tensor(h, t, dst, true, expected_numel > 0, false, stream);
}

// core/safetensors.cpp:316-331 / core/ane_runtime.cpp:197-205
extern "C" void anelm_ane_blob_header(uint8_t* hdr, uint64_t num_elements) {
    memset(hdr, 0, 128);
    hdr[0] = 0x01;
    hdr[4] = 0x02;
    uint8_t* chunk = hdr + 64;
    chunk[0] = 0xEF;
    chunk[1] = 0xBE;
    chunk[2] = 0xAD;
    chunk[3] = 0xDE;
    chunk[4] = 0x01;
    const uint32_t wsize = (uint32_t)(num_elements * 2);   // the reference's (uint32_t) cast
    const uint32_t off = 128;
    memcpy(chunk + 8, &wsize, 4);
    memcpy(chunk + 16, &off, 4);
}

// core/safetensors.cpp:345-383: every BF16 tensor of the file becomes
// <output_dir>/<name with '.' -> '/'>.bin holding the 128-byte header and the
// truncating fp16 convert, done on the GPU.  Chunks flow through two
// pipeline slots: host copy in, H2D, convert, D2H and the file write of the
// chunk two steps back overlap.
extern "C" long anelm_write_ane_blobs(const char* safetensors_path, const char* output_dir, void* stream) {
    anelm_st* h = anelm_st_open(safetensors_path);
    if (!h) return ANELM_ERR_INVALID;
    clear_error();
    if (!output_dir) {
        anelm_st_close(h);
        return fail(ANELM_ERR_INVALID, "write_ane_blobs: null output_dir");
    }
    hipStream_t st = anelm::as_stream(stream);
    long written = 0;
    int rc = ANELM_OK;
    {
        Pipeline p;
        struct Pending {
            FILE* f = nullptr;
            size_t n = 0;
            bool last = false;
            bool busy = false;
        } pend[2];
        auto flush = [&](int k) -> int {
            if (!pend[k].busy) return ANELM_OK;
            hipError_t e = p.wait(k);
            if (e != hipSuccess) return hip_fail(e, "write_ane_blobs");
            if (fwrite(p.hout[k], 1, pend[k].n, pend[k].f) != pend[k].n)
                return fail(ANELM_ERR_INVALID, "write_ane_blobs: write failed: %s", strerror(errno));
            if (pend[k].last && fclose(pend[k].f) != 0)
                return fail(ANELM_ERR_INVALID, "write_ane_blobs: close failed: %s", strerror(errno));
            pend[k] = Pending{};
            return ANELM_OK;
        };
        rc = p.init(true);
        FILE* cur = nullptr;   // the blob being written (closed by the flush of its last chunk)
        uint64_t c = 0;        // global chunk counter: slot = c & 1
        for (size_t ti = 0; rc == ANELM_OK && ti < h->t.size(); ti++) {
            const StTensor& t = h->t[ti];
            if (t.dtype != ANELM_BF16) continue;
            std::string rel = t.name;
            for (char& ch : rel)
                if (ch == '.') ch = '/';
            const std::string path = std::string(output_dir) + "/" + rel + ".bin";
            if (!make_parents(path)) {
                rc = fail(ANELM_ERR_INVALID, "write_ane_blobs: cannot create directories for %s", path.c_str());
                break;
            }
            FILE* f = fopen(path.c_str(), "wb");
            cur = f;
            if (!f) {
                rc = fail(ANELM_ERR_INVALID, "write_ane_blobs: cannot open %s: %s", path.c_str(), strerror(errno));
                break;
            }
            uint8_t hdr[128];
            anelm_ane_blob_header(hdr, (uint64_t)t.numel);
            if (fwrite(hdr, 1, 128, f) != 128) {
                rc = fail(ANELM_ERR_INVALID, "write_ane_blobs: write failed: %s", strerror(errno));
                break;
            }
            if (t.nbytes == 0) {
                cur = nullptr;
                if (fclose(f) != 0) {
                    rc = fail(ANELM_ERR_INVALID, "write_ane_blobs: close failed: %s", strerror(errno));
                    break;
                }
                written++;
                continue;
            }
            const uint8_t* src = h->data + t.offset;
            for (uint64_t off = 0; rc == ANELM_OK && off < t.nbytes; off += kChunkBytes, c++) {
                const int k = (int)(c & 1);
                if ((rc = flush(k)) != ANELM_OK) break;
                const size_t n = (size_t)(t.nbytes - off < kChunkBytes ? t.nbytes - off : kChunkBytes);
                memcpy(p.hin[k], src + off, n);
                hipError_t e = hipMemcpyAsync(p.dev[k], p.hin[k], n, hipMemcpyHostToDevice, st);
                if (e != hipSuccess) {
                    rc = hip_fail(e, "write_ane_blobs H2D");
                    break;
                }
                rc = anelm_bf16_to_f16(reinterpret_cast<uint16_t*>(p.dev[k]), reinterpret_cast<const uint16_t*>(p.dev[k]),
                                       n / 2, stream);
                if (rc) break;
                if ((e = hipMemcpyAsync(p.hout[k], p.dev[k], n, hipMemcpyDeviceToHost, st)) != hipSuccess ||
                    (e = p.record(k, st)) != hipSuccess) {
                    rc = hip_fail(e, "write_ane_blobs D2H");
                    break;
                }
                pend[k] = Pending{f, n, off + n >= t.nbytes, true};
            }
            if (rc == ANELM_OK) {
                written++;
                cur = nullptr;   // now owned by the pending chunks
            }
        }
        // drain in chunk order: the older slot first
        for (int s = 0; s < 2 && rc == ANELM_OK; s++) rc = flush((int)((c + s) & 1));
        if (rc != ANELM_OK) {   // close every file still open, once (rc already holds the error)
            (void)hipStreamSynchronize(st);
            FILE* open_files[3] = {pend[0].busy ? pend[0].f : nullptr, pend[1].busy ? pend[1].f : nullptr, cur};
            for (int a = 0; a < 3; a++) {
                if (!open_files[a]) continue;
                bool seen = false;
                for (int b = 0; b < a; b++) seen = seen || open_files[b] == open_files[a];
                if (!seen) fclose(open_files[a]);
            }
        }
    }
    anelm_st_close(h);
    return rc == ANELM_OK ? written : rc;
}
