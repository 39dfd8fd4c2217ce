// Host side of the C ABI (include/af.h): validation, weight repacking and
// upload, standalone operators, and the generation session that captures the
// whole decode step (the persistent launch of every layer, then the head with greedy
// selection) as one HIP graph replayed per token.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <atomic>
#include <chrono>
#include <cmath>
#include <cstring>
#include <memory>
#include <mutex>
#include <string>
#include <thread>
#include <vector>

#include "../../include/af.h"
#include "af_internal.h"

using namespace af;

namespace {

thread_local std::string g_error;

int fail(int code, std::string msg) {
    g_error = std::move(msg);
    return code;
}

}  // namespace

int af::set_error(int code, std::string msg) { return fail(code, std::move(msg)); }

namespace {

#define HIP_OK(expr, what)                                                                   \
    do {                                                                                     \
        hipError_t e_ = (expr);                                                              \
        if (e_ != hipSuccess) return fail(AF_ERR_DEVICE, std::string(what) + ": " + hipGetErrorString(e_)); \
    } while (0)

using Clock = std::chrono::steady_clock;
double ms_since(Clock::time_point t) { return std::chrono::duration<double, std::milli>(Clock::now() - t).count(); }

// ---- device ---------------------------------------------------------------------------------

std::once_flag g_dev_once;
int g_dev_status = AF_ERR_NO_DEVICE;
std::string g_dev_msg;
hipDeviceProp_t g_props;

int ensure_device() {
    std::call_once(g_dev_once, [] {
        int n = 0;
        if (hipGetDeviceCount(&n) != hipSuccess || n < 1) {
            g_dev_msg = "no HIP device";
            return;
        }
        if (hipGetDeviceProperties(&g_props, 0) != hipSuccess) {
            g_dev_msg = "hipGetDeviceProperties failed";
            return;
        }
        if (std::strncmp(g_props.gcnArchName, "gfx950", 6) != 0) {
            g_dev_msg = std::string("gfx950 (MI355X) required, found ") + g_props.gcnArchName;
            return;
        }
        g_dev_status = AF_OK;
    });
    if (g_dev_status != AF_OK) return fail(g_dev_status, g_dev_msg);
    if (hipSetDevice(0) != hipSuccess) return fail(AF_ERR_DEVICE, "hipSetDevice(0) failed");
    return AF_OK;
}

struct DevMem {
    void* p = nullptr;
    size_t bytes = 0;
    DevMem() = default;
    DevMem(const DevMem&) = delete;
    DevMem& operator=(const DevMem&) = delete;
    DevMem(DevMem&& o) noexcept : p(o.p), bytes(o.bytes) { o.p = nullptr; o.bytes = 0; }
    DevMem& operator=(DevMem&& o) noexcept {
        if (this != &o) {
            reset();
            p = o.p;
            bytes = o.bytes;
            o.p = nullptr;
            o.bytes = 0;
        }
        return *this;
    }
    ~DevMem() { reset(); }
    void reset() {
        if (p) (void)hipFree(p);
        p = nullptr;
        bytes = 0;
    }
    template <typename T>
    T* as() const { return static_cast<T*>(p); }
};

int dev_alloc(DevMem& m, size_t bytes, const char* what) {
    m.reset();
    if (bytes == 0) bytes = 16;
    HIP_OK(hipMalloc(&m.p, bytes), what);
    m.bytes = bytes;
    return AF_OK;
}

int dev_upload(DevMem& m, const void* src, size_t bytes, const char* what) {
    int rc = dev_alloc(m, bytes, what);
    if (rc) return rc;
    HIP_OK(hipMemcpy(m.p, src, bytes, hipMemcpyHostToDevice), what);
    return AF_OK;
}

// Whether this device dispatches the workgroups of a launch to its 8 XCDs in turn, so that
// workgroups b and b + 8 share an XCD: the XCC_ID each workgroup of a 4096-workgroup probe launch
// reads is (XCC_ID of workgroup 0 + b) % 8.  The turn does not restart at XCD 0 with each launch (it
// continues from the previous launch's last workgroup), so only this relative order is checked and
// relied on.  Probed once per process; attention launches rely on it for their XCD-local merge
// (AttnArgs::xcd_local) unless AF_ATTN_XCD_LOCAL=0.
std::once_flag g_xcd_once;
bool g_xcd_rr = false;

bool attn_xcd_local() {
    std::call_once(g_xcd_once, [] {
        constexpr uint32_t kProbe = 4096;
        DevMem map;
        if (dev_alloc(map, (size_t)kProbe * 4, "XCD map") != AF_OK) return;
        std::vector<uint32_t> xcc(kProbe);
        if (step_xcd_map(kProbe, map.as<uint32_t>(), nullptr) != hipSuccess ||
            hipMemcpy(xcc.data(), map.p, (size_t)kProbe * 4, hipMemcpyDeviceToHost) != hipSuccess)
            return;
        bool rr = true;
        for (uint32_t b = 0; b < kProbe; ++b) rr = rr && xcc[b] == (xcc[0] + b) % kXcds;
        g_xcd_rr = rr;
    });
    const char* env = std::getenv("AF_ATTN_XCD_LOCAL");
    return g_xcd_rr && !(env && std::strcmp(env, "0") == 0);
}

// The chunk count attention_kernel derives for `nvis` visible positions (at most cmax chunks of at
// least min_chunk positions, equal lengths but the last).
uint32_t attn_chunks(uint32_t nvis, uint32_t cmax, uint32_t min_chunk) {
    uint32_t chunks = std::min(cmax, (nvis + min_chunk - 1) / min_chunk);
    const uint32_t clen = (nvis + chunks - 1) / chunks;
    return (nvis + clen - 1) / clen;
}

unsigned host_threads() {
    unsigned n = std::thread::hardware_concurrency();
    return std::max(1u, std::min(16u, n ? n : 1u));
}

template <typename F>
void parallel_rows(uint64_t n, F f) {
    const unsigned t = (unsigned)std::min<uint64_t>(host_threads(), std::max<uint64_t>(1, n / 64));
    if (t <= 1) {
        f(0, n);
        return;
    }
    std::vector<std::thread> pool;
    const uint64_t per = (n + t - 1) / t;
    for (unsigned i = 0; i < t; ++i) {
        const uint64_t b = i * per, e = std::min(n, b + per);
        if (b < e) pool.emplace_back(f, b, e);
    }
    for (auto& th : pool) th.join();
}

// ---- validation (mirrors the domain constructors) ---------------------------------------------

bool half_finite(const uint8_t* p) { return ((p[1] << 8 | p[0]) & 0x7C00) != 0x7C00; }

// Q4Matrix::new (crates/domain/src/q4.rs:9-28)
int check_q4(const uint8_t* b, size_t len, uint32_t columns, uint32_t rows, const char* what) {
    if (!b || columns == 0 || rows == 0 || columns % 32 != 0)
        return fail(AF_ERR_INVALID, std::string(what) + ": invalid Q4_0 dimensions");
    if ((uint64_t)(columns / 32) * rows * 18 != (uint64_t)len)
        return fail(AF_ERR_INVALID, std::string(what) + ": inconsistent Q4_0 size");
    for (size_t o = 0; o < len; o += 18)
        if (!half_finite(b + o)) return fail(AF_ERR_INVALID, std::string(what) + ": non-finite Q4_0 scale");
    return AF_OK;
}

// Q6Matrix::new (crates/domain/src/q6.rs:8-20)
int check_q6(const uint8_t* b, size_t len, uint32_t columns, uint32_t rows, const char* what) {
    if (!b || columns == 0 || columns > 65536 || columns % 256 != 0 || rows == 0 || rows > 1000000 ||
        (uint64_t)(columns / 256) * rows * 210 != (uint64_t)len)
        return fail(AF_ERR_INVALID, std::string(what) + ": invalid Q6_K matrix");
    for (size_t o = 0; o < len; o += 210)
        if (!half_finite(b + o + 208)) return fail(AF_ERR_INVALID, std::string(what) + ": invalid Q6_K matrix");
    return AF_OK;
}

// RmsNorm::new (crates/domain/src/rms_norm.rs:8-16)
int check_norm(const af_rms_norm& n, uint32_t expect, const char* what) {
    if (!n.weights || n.len == 0 || n.len > 65536)
        return fail(AF_ERR_INVALID, std::string(what) + ": invalid RMSNorm weights (1 to 65536 finite values required)");
    for (uint32_t i = 0; i < n.len; ++i)
        if (!std::isfinite(n.weights[i]))
            return fail(AF_ERR_INVALID, std::string(what) + ": invalid RMSNorm weights (1 to 65536 finite values required)");
    if (!std::isfinite(n.epsilon) || n.epsilon <= 0.0f)
        return fail(AF_ERR_INVALID, std::string(what) + ": RMSNorm epsilon must be finite and positive");
    if (expect && n.len != expect) return fail(AF_ERR_INVALID, std::string(what) + ": RMSNorm width mismatch");
    return AF_OK;
}

// Rope::new (crates/domain/src/rope.rs:11-34)
int check_rope(const af_rope_params& r) {
    if (r.width == 0 || r.width > 65536 || r.width % 2 != 0 || !r.factors || !std::isfinite(r.base) ||
        r.base <= 1.0 || r.context == 0)
        return fail(AF_ERR_INVALID, "invalid RoPE parameters");
    for (uint32_t i = 0; i < r.width / 2; ++i)
        if (!std::isfinite(r.factors[i]) || r.factors[i] <= 0.0f) return fail(AF_ERR_INVALID, "invalid RoPE parameters");
    return AF_OK;
}

// AttentionConfig::new (crates/domain/src/attention.rs:11-35)
int check_attention(const af_attention_config& c) {
    if (c.q_heads == 0 || c.kv_heads == 0 || c.width == 0 || c.q_heads % c.kv_heads != 0 || !std::isfinite(c.scale) ||
        c.scale <= 0.0f || (uint64_t)c.q_heads * c.width > 0xFFFFFFFFull)
        return fail(AF_ERR_INVALID, "invalid attention configuration");
    return AF_OK;
}

// Kernel shape limits (in addition to the reference's own validation).
int check_supported_q4(uint32_t columns, const char* what) {
    if (columns > 16384) return fail(AF_ERR_INVALID, std::string(what) + ": Q4_0 columns above 16384 are not supported");
    return AF_OK;
}
int check_supported_attention(const af_attention_config& c) {
    const uint32_t g = c.q_heads / c.kv_heads;
    if (c.width != 256 && c.width != 512) return fail(AF_ERR_INVALID, "attention head width must be 256 or 512");
    if (c.width == 256 && g != 1 && g != 2 && g != 4)
        return fail(AF_ERR_INVALID, "query heads per KV head must be 1, 2 or 4 at width 256");
    if (c.width == 512 && g != 1 && g != 2 && g != 4 && g != 8 && g != 16)
        return fail(AF_ERR_INVALID, "query heads per KV head must be 1, 2, 4, 8 or 16 at width 512");
    return AF_OK;
}

std::vector<double> inverse_frequencies(const af_rope_params& r) {
    // Rope::new (crates/domain/src/rope.rs:25-29): base^(-2 i / width) / factor_i in f64.
    std::vector<double> f(r.width / 2);
    for (uint32_t i = 0; i < r.width / 2; ++i)
        f[i] = std::pow(r.base, -2.0 * (double)i / (double)r.width) / (double)r.factors[i];
    return f;
}

// ---- repacking --------------------------------------------------------------------------------

struct Q4Dev {
    DevMem codes, scales;
    uint32_t rows = 0, columns = 0;
    Q4View view() const {
        const uint32_t B = columns / 32;
        return Q4View{codes.as<uint8_t>(), scales.as<uint16_t>(), rows, B, (B + 3) / 4};
    }
};

// Concatenates the rows of several Q4_0 matrices (same columns) into one device matrix in the
// tiled layout of Q4View: 16-row tiles x 4-block super-tiles, zero-padded.
int upload_q4(Q4Dev& d, const std::vector<af_matrix>& parts) {
    const uint32_t columns = parts[0].columns, B = columns / 32, nst = (B + 3) / 4;
    uint64_t rows = 0;
    for (auto& p : parts) rows += p.rows;
    const uint64_t tiles = (rows + 15) / 16;
    std::vector<uint8_t> codes(tiles * nst * 1024, 0);
    std::vector<uint16_t> scales(tiles * nst * 64, 0);
    uint64_t r0 = 0;
    for (auto& p : parts) {
        const uint8_t* src = p.bytes;
        parallel_rows(p.rows, [&](uint64_t b, uint64_t e) {
            for (uint64_t r = b; r < e; ++r) {
                const uint64_t R = r0 + r, rt = R / 16, rr = R % 16;
                for (uint32_t k = 0; k < B; ++k) {
                    const uint8_t* blk = src + (r * B + k) * 18;
                    const uint64_t tile = rt * nst + k / 4;
                    std::memcpy(&codes[(tile * 64 + (k & 3) * 16 + rr) * 16], blk + 2, 16);
                    scales[tile * 64 + (k & 3) * 16 + rr] = (uint16_t)(blk[0] | (blk[1] << 8));
                }
            }
        });
        r0 += p.rows;
    }
    int rc = dev_upload(d.codes, codes.data(), codes.size(), "Q4_0 codes upload");
    if (rc) return rc;
    rc = dev_upload(d.scales, scales.data(), scales.size() * 2, "Q4_0 scales upload");
    if (rc) return rc;
    d.rows = (uint32_t)rows;
    d.columns = columns;
    return AF_OK;
}

struct Q6Dev {
    DevMem a, b, h, s, d, t;
    uint32_t rows = 0, columns = 0;
    Q6View view() const {
        return Q6View{a.as<uint8_t>(), b.as<uint8_t>(), h.as<uint8_t>(), s.as<uint32_t>(), d.as<uint16_t>(), rows,
                      columns / 64, t.as<uint8_t>()};
    }
};

// Head records (kQ6Rec) from GGUF Q6_K super-blocks: rows padded to a multiple of 16 with zero
// codes and scales.  Weight e of a super-block (q6.rs layout): low nibble of ql[64 (e / 128) +
// 32 (e / 32 % 2) + e % 32] (the high nibble when e % 128 >= 64), high bits (qh[32 (e / 128) +
// e % 32] >> 2 (e % 128 / 32)) & 3, scale sc[e / 16], d at byte 208.
std::vector<uint8_t> q6_head_records(const uint8_t* src, uint32_t columns, uint32_t rows) {
    const uint64_t sblocks = columns / 256, tiles = (rows + 15) / 16;
    std::vector<uint8_t> T(tiles * sblocks * kQ6Rec, 0);
    parallel_rows(tiles * sblocks, [&](uint64_t b0, uint64_t e0) {
        for (uint64_t i = b0; i < e0; ++i) {
            const uint64_t tile = i / sblocks, sbk = i % sblocks;
            uint8_t* rec = &T[i * kQ6Rec];
            for (uint32_t r = 0; r < 16; ++r) {
                const uint64_t row = tile * 16 + r;
                if (row >= rows) continue;
                const uint8_t* blk = src + (row * sblocks + sbk) * 210;
                const uint8_t *ql = blk, *qh = blk + 128, *sc = blk + 192;
                rec[3328 + 2 * r] = blk[208];
                rec[3329 + 2 * r] = blk[209];
                for (uint32_t g = 0; g < 4; ++g) {
                    const uint32_t lane = 16 * g + r;
                    for (uint32_t kb = 0; kb < 4; ++kb) {
                        uint8_t c[16];
                        for (uint32_t j = 0; j < 16; ++j) {
                            const uint32_t e = 64 * kb + 16 * g + j, l = e % 128;
                            const uint8_t lo = ql[64 * (e / 128) + 32 * (l / 32 % 2) + l % 32];
                            const uint8_t nib = l >= 64 ? (uint8_t)(lo >> 4) : (uint8_t)(lo & 15);
                            const uint8_t hi = (uint8_t)((qh[32 * (e / 128) + l % 32] >> (2 * (l / 32))) & 3);
                            c[j] = (uint8_t)(nib | (hi << 4));
                        }
                        uint8_t w[12];
                        for (uint32_t b = 0; b < 4; ++b) {
                            w[b] = (uint8_t)((c[b] & 15) | ((c[4 + b] & 15) << 4));
                            w[4 + b] = (uint8_t)((c[8 + b] & 15) | ((c[12 + b] & 15) << 4));
                            w[8 + b] = (uint8_t)((c[b] >> 4) | ((c[4 + b] >> 4) << 2) | ((c[8 + b] >> 4) << 4) |
                                                 ((c[12 + b] >> 4) << 6));
                        }
                        for (uint32_t q = 0; q < 3; ++q) {  // dwords 3 kb .. 3 kb + 2 of the lane
                            const uint32_t dw = 3 * kb + q;
                            std::memcpy(rec + (dw / 4) * 1024 + lane * 16 + (dw % 4) * 4, w + 4 * q, 4);
                        }
                        rec[3072 + lane * 4 + kb] = sc[4 * kb + g];
                    }
                }
            }
        }
    });
    return T;
}

int upload_q6(Q6Dev& dv, const uint8_t* src, uint32_t columns, uint32_t rows) {
    const uint64_t units = columns / 64, sblocks = columns / 256;
    std::vector<uint8_t> A(rows * units * 16), B(rows * units * 16), H(rows * units * 16);
    std::vector<uint32_t> S(rows * units);
    std::vector<uint16_t> D(rows * sblocks);
    parallel_rows((uint64_t)rows * sblocks, [&](uint64_t b0, uint64_t e0) {
        for (uint64_t i = b0; i < e0; ++i) {
            const uint8_t* blk = src + i * 210;
            const uint8_t *ql = blk, *qh = blk + 128, *sc = blk + 192;
            D[i] = (uint16_t)(blk[208] | (blk[209] << 8));
            for (int g = 0; g < 2; ++g)
                for (int hh = 0; hh < 2; ++hh) {
                    const uint64_t u = i * 4 + g * 2 + hh;  // row * units + unit
                    std::memcpy(&A[u * 16], ql + 64 * g + 16 * hh, 16);
                    std::memcpy(&B[u * 16], ql + 64 * g + 32 + 16 * hh, 16);
                    std::memcpy(&H[u * 16], qh + 32 * g + 16 * hh, 16);
                    uint32_t w = 0;
                    for (int q = 0; q < 4; ++q) w |= (uint32_t)sc[8 * g + 2 * q + hh] << (8 * q);
                    S[u] = w;
                }
        }
    });
    int rc;
    if ((rc = dev_upload(dv.a, A.data(), A.size(), "Q6_K upload"))) return rc;
    if ((rc = dev_upload(dv.b, B.data(), B.size(), "Q6_K upload"))) return rc;
    if ((rc = dev_upload(dv.h, H.data(), H.size(), "Q6_K upload"))) return rc;
    if ((rc = dev_upload(dv.s, S.data(), S.size() * 4, "Q6_K upload"))) return rc;
    if ((rc = dev_upload(dv.d, D.data(), D.size() * 2, "Q6_K upload"))) return rc;
    const std::vector<uint8_t> T = q6_head_records(src, columns, rows);
    if ((rc = dev_upload(dv.t, T.data(), T.size(), "Q6_K upload"))) return rc;
    dv.rows = rows;
    dv.columns = columns;
    return AF_OK;
}

float median_of(std::vector<float> t) {
    if (t.empty()) return 0.0f;
    std::sort(t.begin(), t.end());
    const size_t n = t.size();
    return n % 2 ? t[n / 2] : 0.5f * (t[n / 2 - 1] + t[n / 2]);
}

// Scratch for the standalone head / attention entry points (grown on demand, never shrunk).
struct Scratch {
    std::mutex mu;
    DevMem head_partial, head_counter, attn_part, attn_counters;
    DevMem batch_image, batch_part;     // digit image and split-K partials of af_q4_gemm
    DevMem attn_freq;                   // the last RoPE inverse frequencies of af_attention_decode
    std::vector<double> attn_freq_host; // their host copy (re-uploaded only when they change)
};
Scratch g_scratch;

int grow(DevMem& m, size_t bytes, bool zero, const char* what) {
    if (m.bytes >= bytes) return AF_OK;
    int rc = dev_alloc(m, bytes, what);
    if (rc) return rc;
    if (zero) HIP_OK(hipMemset(m.p, 0, bytes), what);
    return AF_OK;
}

// Scratch of the allocation-free head entry point (af_q6_gemv_argmax_noalloc): a fixed array in
// the library's device memory, one copy per GPU, held until the process ends.  Bytes [0, 256) hold
// the completion counter, then one 16-byte argmax partial per workgroup.  Its device address is
// looked up once per device (with that device current) and kept: in host code `scratch` names a
// host-side stand-in, never the device copy.
constexpr size_t kNoAllocScratchBytes = AF_NOALLOC_SCRATCH_BYTES;
constexpr size_t kNoAllocCounterBytes = 256;
static __device__ __align__(256) uint8_t scratch[kNoAllocScratchBytes];
constexpr int kMaxDevices = 64;
std::once_flag g_noalloc_once[kMaxDevices];
void* g_noalloc_ptr[kMaxDevices];
hipError_t g_noalloc_status[kMaxDevices];

int noalloc_scratch(void** out) {
    int dev = -1;
    HIP_OK(hipGetDevice(&dev), "current device");
    if (dev < 0 || dev >= kMaxDevices) return fail(AF_ERR_DEVICE, "device index outside the scratch table");
    std::call_once(g_noalloc_once[dev], [dev] {
        g_noalloc_status[dev] = hipGetSymbolAddress(&g_noalloc_ptr[dev], HIP_SYMBOL(scratch));
    });
    HIP_OK(g_noalloc_status[dev], "scratch array address");
    *out = g_noalloc_ptr[dev];
    return AF_OK;
}

}  // namespace

// ================================================================================================
// C ABI
// ================================================================================================

struct af_q4 {
    Q4Dev m;
};
struct af_q6 {
    Q6Dev m;
};

extern "C" {

const char* af_last_error(void) { return g_error.c_str(); }

int af_device_query(af_device_info* out) {
    if (!out) return fail(AF_ERR_INVALID, "null output");
    int rc = ensure_device();
    if (rc) return rc;
    std::memset(out, 0, sizeof(*out));
    std::snprintf(out->name, sizeof(out->name), "%s", g_props.name);
    std::snprintf(out->arch, sizeof(out->arch), "%s", g_props.gcnArchName);
    out->compute_units = g_props.multiProcessorCount;
    size_t fr = 0, tot = 0;
    HIP_OK(hipMemGetInfo(&fr, &tot), "hipMemGetInfo");
    out->free_memory_bytes = fr;
    out->total_memory_bytes = tot;
    return AF_OK;
}

int af_q4_upload(const uint8_t* q4, size_t len, uint32_t columns, uint32_t rows, af_q4** out) {
    if (!out) return fail(AF_ERR_INVALID, "null output");
    *out = nullptr;
    int rc = check_q4(q4, len, columns, rows, "Q4_0 matrix");
    if (rc) return rc;
    if ((rc = check_supported_q4(columns, "Q4_0 matrix"))) return rc;
    if ((rc = ensure_device())) return rc;
    auto m = std::make_unique<af_q4>();
    if ((rc = upload_q4(m->m, {af_matrix{q4, len, columns, rows}}))) return rc;
    *out = m.release();
    return AF_OK;
}

void af_q4_free(af_q4* m) { delete m; }

int af_q4_gemv(const af_q4* m, const float* x, float* y, void* stream) {
    if (!m || !x || !y) return fail(AF_ERR_INVALID, "null argument");
    Q4Args a{};
    a.w = m->m.view();
    a.in.x = x;
    a.y = y;
    HIP_OK(launch_q4_gemv(a, IN_PLAIN, OUT_PLAIN, m->m.rows, (hipStream_t)stream), "Q4_0 GEMV launch");
    return AF_OK;
}

int af_q4_gemm(const af_q4* m, const float* x, uint32_t tokens, float* y, void* stream) {
    if (!m || !x || !y) return fail(AF_ERR_INVALID, "null argument");
    if (tokens == 0 || tokens > kBatchMax)
        return fail(AF_ERR_INVALID, "batched GEMV takes 1 to " + std::to_string(kBatchMax) + " vectors");
    const Q4View w = m->m.view();
    std::lock_guard<std::mutex> lock(g_scratch.mu);
    int rc;
    if ((rc = grow(g_scratch.batch_image, batch_image_bytes(w.blocks, kBatchMax), false, "batch digit image")))
        return rc;
    if ((rc = grow(g_scratch.batch_part, batch_gemm_part_bytes(w.rows, w.blocks, kBatchMax, false) + 4, false,
                   "batch partials")))
        return rc;
    const hipStream_t s = (hipStream_t)stream;
    BatchIn in{};
    in.mode = BI_PLAIN;
    in.T = tokens;
    in.K = w.blocks * 32;
    in.stride = in.K;
    in.x = x;
    in.img = g_scratch.batch_image.as<int8_t>();
    HIP_OK(launch_batch_input(in, s), "batched GEMV input digits");
    BatchGemm g{};
    g.w = w;
    g.img = in.img;
    g.T = tokens;
    g.y = y;
    g.y_stride = w.rows;
    g.part = g_scratch.batch_part.as<float>();
    HIP_OK(launch_batch_gemm(g, false, s), "batched GEMV launch");
    return AF_OK;
}

int af_q6_upload(const uint8_t* q6, size_t len, uint32_t columns, uint32_t rows, af_q6** out) {
    if (!out) return fail(AF_ERR_INVALID, "null output");
    *out = nullptr;
    int rc = check_q6(q6, len, columns, rows, "Q6_K matrix");
    if (rc) return rc;
    if (columns > 4096) return fail(AF_ERR_INVALID, "Q6_K columns above 4096 are not supported");
    if ((rc = ensure_device())) return rc;
    auto m = std::make_unique<af_q6>();
    if ((rc = upload_q6(m->m, q6, columns, rows))) return rc;
    *out = m.release();
    return AF_OK;
}

void af_q6_free(af_q6* m) { delete m; }

int af_q6_gemv_argmax(const af_q6* m, const float* x, float* logits, uint32_t* result, void* stream) {
    if (!m || !x || !result) return fail(AF_ERR_INVALID, "null argument");
    std::lock_guard<std::mutex> lock(g_scratch.mu);
    const uint32_t grid = head_grid(m->m.rows);
    int rc;
    if ((rc = grow(g_scratch.head_partial, (size_t)grid * sizeof(uint4), false, "head scratch"))) return rc;
    if ((rc = grow(g_scratch.head_counter, 256, true, "head counter"))) return rc;
    HeadArgs a{};
    a.w = m->m.view();
    a.in.x = x;
    a.logits = logits;
    a.partial = g_scratch.head_partial.as<uint4>();
    a.counter = g_scratch.head_counter.as<uint32_t>();
    a.result = result;
    HIP_OK(launch_head(a, IN_PLAIN, grid, (hipStream_t)stream), "Q6_K head launch");
    return AF_OK;
}

int af_q6_gemv_argmax_noalloc(const af_q6* m, const float* x, float* logits, uint32_t* result, void* stream) {
    if (!m || !x || !result) return fail(AF_ERR_INVALID, "null argument");
    const uint32_t grid = head_grid(m->m.rows);
    const size_t need = kNoAllocCounterBytes + (size_t)grid * sizeof(uint4);
    if (need > kNoAllocScratchBytes)
        return fail(AF_ERR_INVALID, "Q6_K head needs " + std::to_string(need) + " bytes of scratch, above the " +
                                        std::to_string(kNoAllocScratchBytes) + "-byte allocation-free array");
    void* base = nullptr;
    int rc = noalloc_scratch(&base);
    if (rc) return rc;
    uint8_t* p = static_cast<uint8_t*>(base);
    HeadArgs a{};
    a.w = m->m.view();
    a.in.x = x;
    a.logits = logits;
    a.partial = reinterpret_cast<uint4*>(p + kNoAllocCounterBytes);
    a.counter = reinterpret_cast<uint32_t*>(p);
    a.result = result;
    // the array keeps the last call's contents: the counter must start at zero
    HIP_OK(launch_zero_words(a.counter, 1, (hipStream_t)stream), "scratch clear");
    HIP_OK(launch_head(a, IN_PLAIN, grid, (hipStream_t)stream), "Q6_K head launch");
    return AF_OK;
}

int af_rmsnorm(const float* x, const float* weights, float* y, uint32_t width, uint32_t vectors, float eps,
               void* stream) {
    if (!x || !weights || !y || width == 0 || vectors == 0) return fail(AF_ERR_INVALID, "invalid RMSNorm arguments");
    if (!std::isfinite(eps) || eps <= 0.0f) return fail(AF_ERR_INVALID, "RMSNorm epsilon must be finite and positive");
    HIP_OK(launch_rmsnorm(x, weights, y, width, vectors, eps, (hipStream_t)stream), "RMSNorm launch");
    return AF_OK;
}

int af_softcap(const float* x, float* y, size_t n, float cap, void* stream) {
    if (!x || !y || n == 0) return fail(AF_ERR_INVALID, "invalid softcap arguments");
    if (!std::isfinite(cap) || cap <= 0.0f) return fail(AF_ERR_INVALID, "Softcapping invalide");  // q6.rs:67-69
    HIP_OK(launch_softcap(x, y, n, cap, (hipStream_t)stream), "softcap launch");
    return AF_OK;
}

int af_matvec_run(const uint8_t* q4, size_t len, uint32_t columns, uint32_t rows, const float* inputs,
                  uint32_t n_inputs, uint32_t timed_repetitions, float* outputs, float* median_ms) {
    int rc = check_q4(q4, len, columns, rows, "Q4_0 matrix");
    if (rc) return rc;
    if ((rc = check_supported_q4(columns, "Q4_0 matrix"))) return rc;
    if (!inputs || !outputs || n_inputs == 0) return fail(AF_ERR_INVALID, "invalid input vectors");
    for (uint64_t i = 0; i < (uint64_t)n_inputs * columns; ++i)
        if (!std::isfinite(inputs[i])) return fail(AF_ERR_INVALID, "invalid input vector");
    if ((rc = ensure_device())) return rc;
    Q4Dev m;
    if ((rc = upload_q4(m, {af_matrix{q4, len, columns, rows}}))) return rc;
    DevMem x, y;
    if ((rc = dev_alloc(x, (size_t)columns * 4, "input"))) return rc;
    if ((rc = dev_alloc(y, (size_t)rows * 4, "output"))) return rc;
    hipEvent_t e0, e1;
    HIP_OK(hipEventCreate(&e0), "event");
    HIP_OK(hipEventCreate(&e1), "event");
    std::vector<float> times;
    Q4Args a{};
    a.w = m.view();
    a.in.x = x.as<float>();
    a.y = y.as<float>();
    int status = AF_OK;
    for (uint32_t v = 0; v < n_inputs && !status; ++v) {
        if (hipMemcpy(x.p, inputs + (size_t)v * columns, (size_t)columns * 4, hipMemcpyHostToDevice) != hipSuccess) {
            status = fail(AF_ERR_DEVICE, "input upload");
            break;
        }
        const uint32_t execs = v + 1 == n_inputs ? 1 + timed_repetitions : 1;
        for (uint32_t r = 0; r < execs; ++r) {
            hipError_t e = hipEventRecord(e0, 0);
            if (e == hipSuccess) e = launch_q4_gemv(a, IN_PLAIN, OUT_PLAIN, rows, 0);
            if (e == hipSuccess) e = hipEventRecord(e1, 0);
            if (e == hipSuccess) e = hipEventSynchronize(e1);
            if (e != hipSuccess) {
                status = fail(AF_ERR_DEVICE, std::string("matvec launch: ") + hipGetErrorString(e));
                break;
            }
            if (v + 1 == n_inputs && r > 0) {
                float t = 0;
                (void)hipEventElapsedTime(&t, e0, e1);
                times.push_back(t);
            }
        }
        if (!status && hipMemcpy(outputs + (size_t)v * rows, y.p, (size_t)rows * 4, hipMemcpyDeviceToHost) != hipSuccess)
            status = fail(AF_ERR_DEVICE, "output download");
    }
    (void)hipEventDestroy(e0);
    (void)hipEventDestroy(e1);
    if (median_ms) *median_ms = median_of(times);
    return status;
}

int af_rmsnorm_run(const float* weights, uint32_t width, float eps, const float* inputs, uint32_t vectors,
                   uint32_t timed_repetitions, float* outputs, float* median_ms) {
    int rc = check_norm(af_rms_norm{weights, width, eps}, 0, "RMSNorm");
    if (rc) return rc;
    if (!inputs || !outputs || vectors == 0) return fail(AF_ERR_INVALID, "invalid RMSNorm input");
    for (uint64_t i = 0; i < (uint64_t)vectors * width; ++i)
        if (!std::isfinite(inputs[i])) return fail(AF_ERR_INVALID, "invalid RMSNorm input");
    if ((rc = ensure_device())) return rc;
    DevMem x, w, y;
    const size_t n = (size_t)vectors * width * 4;
    if ((rc = dev_upload(x, inputs, n, "RMSNorm input"))) return rc;
    if ((rc = dev_upload(w, weights, (size_t)width * 4, "RMSNorm weights"))) return rc;
    if ((rc = dev_alloc(y, n, "RMSNorm output"))) return rc;
    hipEvent_t e0, e1;
    HIP_OK(hipEventCreate(&e0), "event");
    HIP_OK(hipEventCreate(&e1), "event");
    std::vector<float> times;
    int status = AF_OK;
    for (uint32_t r = 0; r < 1 + timed_repetitions; ++r) {
        hipError_t e = hipEventRecord(e0, 0);
        if (e == hipSuccess) e = launch_rmsnorm(x.as<float>(), w.as<float>(), y.as<float>(), width, vectors, eps, 0);
        if (e == hipSuccess) e = hipEventRecord(e1, 0);
        if (e == hipSuccess) e = hipEventSynchronize(e1);
        if (e != hipSuccess) {
            status = fail(AF_ERR_DEVICE, std::string("RMSNorm launch: ") + hipGetErrorString(e));
            break;
        }
        if (r > 0) {
            float t = 0;
            (void)hipEventElapsedTime(&t, e0, e1);
            times.push_back(t);
        }
    }
    if (!status && hipMemcpy(outputs, y.p, n, hipMemcpyDeviceToHost) != hipSuccess)
        status = fail(AF_ERR_DEVICE, "RMSNorm download");
    (void)hipEventDestroy(e0);
    (void)hipEventDestroy(e1);
    if (median_ms) *median_ms = median_of(times);
    return status;
}

}  // extern "C"

// ---- FFN ---------------------------------------------------------------------------------------

struct af_ffn {
    Q4Dev gate, up, down;
    DevMem pre, post, act, act_img, mid;  // act_img: the down GEMV's input as its digit image
    float pre_eps = 0, post_eps = 0, scale = 1;
    bool has_post = false;
    uint32_t hidden = 0, intermediate = 0;
};

extern "C" {

int af_ffn_create(const af_ffn_weights* w, af_ffn** out) {
    if (!w || !out) return fail(AF_ERR_INVALID, "null argument");
    *out = nullptr;
    // Ffn::new (crates/domain/src/ffn.rs:70-98)
    const uint32_t hidden = w->gate.columns, inter = w->gate.rows;
    int rc;
    if ((rc = check_q4(w->gate.bytes, w->gate.len, w->gate.columns, w->gate.rows, "FFN gate"))) return rc;
    if ((rc = check_q4(w->up.bytes, w->up.len, w->up.columns, w->up.rows, "FFN up"))) return rc;
    if ((rc = check_q4(w->down.bytes, w->down.len, w->down.columns, w->down.rows, "FFN down"))) return rc;
    if (w->up.columns != hidden || w->up.rows != inter || w->down.columns != inter || w->down.rows != hidden ||
        !std::isfinite(w->layer_scale))
        return fail(AF_ERR_INVALID, "incompatible FFN dimensions or scale");
    if ((rc = check_norm(w->pre, hidden, "FFN pre-norm"))) return rc;
    const bool has_post = w->post.weights != nullptr;
    if (has_post && (rc = check_norm(w->post, hidden, "FFN post-norm"))) return rc;
    if ((rc = check_supported_q4(hidden, "FFN gate"))) return rc;
    if ((rc = check_supported_q4(inter, "FFN down"))) return rc;
    if ((rc = ensure_device())) return rc;
    auto f = std::make_unique<af_ffn>();
    if ((rc = upload_q4(f->gate, {w->gate}))) return rc;
    if ((rc = upload_q4(f->up, {w->up}))) return rc;
    if ((rc = upload_q4(f->down, {w->down}))) return rc;
    if ((rc = dev_upload(f->pre, w->pre.weights, (size_t)hidden * 4, "FFN norm"))) return rc;
    if (has_post && (rc = dev_upload(f->post, w->post.weights, (size_t)hidden * 4, "FFN norm"))) return rc;
    if ((rc = dev_alloc(f->act, (size_t)inter * 4, "FFN activations"))) return rc;
    const size_t img = (size_t)(inter + 127) / 128 * kStepImg;  // blocks past the activations stay zero
    if ((rc = dev_alloc(f->act_img, img, "FFN activation digits"))) return rc;
    HIP_OK(hipMemset(f->act_img.p, 0, img), "FFN activation digits clear");
    if ((rc = dev_alloc(f->mid, (size_t)hidden * 4, "FFN down output"))) return rc;
    f->pre_eps = w->pre.epsilon;
    f->post_eps = w->post.epsilon;
    f->scale = w->layer_scale;
    f->has_post = has_post;
    f->hidden = hidden;
    f->intermediate = inter;
    *out = f.release();
    return AF_OK;
}

void af_ffn_free(af_ffn* f) { delete f; }

int af_ffn_run(af_ffn* f, const float* x, float* y, void* stream) {
    if (!f || !x || !y) return fail(AF_ERR_INVALID, "null argument");
    hipStream_t s = (hipStream_t)stream;
    Q4Args g{};
    g.w = f->gate.view();
    g.w2 = f->up.view();
    g.in.x = x;
    g.in.w_n = f->pre.as<float>();
    g.in.eps_n = f->pre_eps;
    g.y = f->act.as<float>();
    g.dig_out = f->act_img.as<int8_t>();  // the down GEMV's input, as its digit image
    HIP_OK(launch_q4_gemv(g, IN_NORM, OUT_GELU, f->intermediate, s), "FFN gate/up launch");
    Q4Args d{};
    d.w = f->down.view();
    d.in.dig = f->act_img.as<int8_t>();
    if (!f->has_post && f->scale == 1.0f) {  // down + residual in the GEMV epilogue
        d.y = y;
        d.add = x;
        HIP_OK(launch_q4_gemv(d, IN_DIGITS, OUT_ADD, f->hidden, s), "FFN down launch");
        return AF_OK;
    }
    d.y = f->mid.as<float>();
    HIP_OK(launch_q4_gemv(d, IN_DIGITS, OUT_PLAIN, f->hidden, s), "FFN down launch");
    InputStage r{};
    r.x = f->mid.as<float>();
    r.res = x;
    r.w_a = f->has_post ? f->post.as<float>() : nullptr;
    r.eps_a = f->post_eps;
    r.scale = f->scale;
    HIP_OK(launch_resid(r, f->hidden, y, s), "FFN tail launch");
    return AF_OK;
}

int af_attention_decode(const af_attention_args* p, void* stream) {
    if (!p || !p->q || !p->k || !p->v || !p->q_norm || !p->k_norm || !p->k_cache || !p->v_cache || !p->out)
        return fail(AF_ERR_INVALID, "null attention argument");
    int rc;
    if ((rc = check_attention(p->config))) return rc;
    if ((rc = check_rope(p->rope))) return rc;
    if ((rc = check_supported_attention(p->config))) return rc;
    if (p->rope.width != p->config.width) return fail(AF_ERR_INVALID, "RoPE width differs from head width");
    if (p->position >= p->rope.context) return fail(AF_ERR_INVALID, "position outside the RoPE context");
    const uint32_t nvis = p->config.window ? std::min(p->position + 1, p->config.window) : p->position + 1;
    if (p->ring < nvis || p->ring == 0) return fail(AF_ERR_INVALID, "KV ring smaller than the visible range");
    if ((uint64_t)p->ring * p->config.width * 2 > 0x7FFF0000ull)  // addressed with 32-bit byte offsets
        return fail(AF_ERR_INVALID, "KV ring above 2 GiB per KV head");
    for (float e : {p->q_eps, p->k_eps, p->v_eps})
        if (!std::isfinite(e) || e <= 0.0f) return fail(AF_ERR_INVALID, "epsilon must be finite and positive");
    if ((rc = ensure_device())) return rc;
    const uint32_t group = p->config.q_heads / p->config.kv_heads, D = p->config.width;
    if (nvis > kAttnMaxChunks * kAttnMaxChunkLen) return fail(AF_ERR_INVALID, "visible range above 131072 tokens");
    const uint32_t cmax = kAttnMaxChunks;
    const bool xl = attn_xcd_local();
    std::lock_guard<std::mutex> lock(g_scratch.mu);
    if ((rc = grow(g_scratch.attn_part, (size_t)p->config.kv_heads * cmax * group * attn_part_row(D) * 4, false, "attention scratch")))
        return rc;
    if ((rc = grow(g_scratch.attn_counters, (size_t)std::max<uint32_t>(64, p->config.q_heads) * 4, true,
                   "attention counters")))
        return rc;
    // inverse frequencies: kept on the device and re-uploaded only when the RoPE parameters change
    // (after the device drains, so no launch still reads the old ones); repeated calls with the
    // same parameters enqueue one kernel and nothing else
    std::vector<double> f = inverse_frequencies(p->rope);
    if (f != g_scratch.attn_freq_host) {
        HIP_OK(hipDeviceSynchronize(), "attention frequencies");
        if ((rc = grow(g_scratch.attn_freq, f.size() * 8, false, "RoPE frequencies"))) return rc;
        HIP_OK(hipMemcpy(g_scratch.attn_freq.p, f.data(), f.size() * 8, hipMemcpyHostToDevice), "RoPE frequencies");
        g_scratch.attn_freq_host = f;
    }
    AttnArgs a{};
    a.q_raw = p->q;
    a.k_raw = p->k;
    a.v_raw = p->v;
    a.q_norm = p->q_norm;
    a.k_norm = p->k_norm;
    a.q_eps = p->q_eps;
    a.k_eps = p->k_eps;
    a.v_eps = p->v_eps;
    a.v_norm = p->v_norm;
    a.inv_freq = g_scratch.attn_freq.as<double>();
    a.kcache = p->k_cache;
    a.vcache = p->v_cache;
    a.ring = p->ring;
    a.window = p->config.window;
    a.scale = p->config.scale;
    a.position = p->position;
    a.out = p->out;
    a.part = g_scratch.attn_part.as<float>();
    a.counters = g_scratch.attn_counters.as<uint32_t>();
    a.cmax = attn_chunks(nvis, cmax, kAttnMinChunk);  // the position is known: a block per chunk
    a.min_chunk = kAttnMinChunk;
    a.kv_heads = p->config.kv_heads;
    a.group = group;
    a.xcd_local = xl ? 1u : 0u;
    HIP_OK(launch_attention(a, group, D, (hipStream_t)stream), "attention launch");
    return AF_OK;
}

}  // extern "C"

// ---- generation session --------------------------------------------------------------------------

namespace {

struct LayerDev {
    Q4Dev qkv, o, gate, up, down;
    DevMem input_norm, q_norm, k_norm, post_attn, ffn_norm, post_ffn, inv_freq, kcache, vcache;
    float input_eps = 0, q_eps = 0, k_eps = 0, post_attn_eps = 0, ffn_eps = 0, post_ffn_eps = 0;
    float layer_scale = 1, scale = 1;
    uint32_t q_heads = 0, kv_heads = 0, width = 0, window = 0, ring = 0, qn = 0, kn = 0;
    bool shared_v = false, v_norm = false;
};

int validate_layer(const af_layer_weights& w, uint32_t hidden, uint32_t capacity, uint32_t index) {
    const std::string tag = "layer " + std::to_string(index);
    int rc;
    for (int i = 0; i < 3; ++i)
        if ((rc = check_q4(w.matrices[i].bytes, w.matrices[i].len, w.matrices[i].columns, w.matrices[i].rows,
                           (tag + " qkv").c_str())))
            return rc;
    if ((rc = check_q4(w.output.bytes, w.output.len, w.output.columns, w.output.rows, (tag + " output").c_str())))
        return rc;
    const af_ffn_weights& f = w.ffn;
    if ((rc = check_q4(f.gate.bytes, f.gate.len, f.gate.columns, f.gate.rows, (tag + " gate").c_str()))) return rc;
    if ((rc = check_q4(f.up.bytes, f.up.len, f.up.columns, f.up.rows, (tag + " up").c_str()))) return rc;
    if ((rc = check_q4(f.down.bytes, f.down.len, f.down.columns, f.down.rows, (tag + " down").c_str()))) return rc;
    if ((rc = check_rope(w.rope))) return rc;
    if ((rc = check_attention(w.attention))) return rc;
    const uint32_t hw = w.rope.width;
    // stack.rs:60-84 (validate)
    if (capacity == 0 || capacity > AF_MAX_CONTEXT || capacity > w.rope.context || w.input_norm.len != hidden ||
        w.matrices[0].columns != hidden || w.matrices[1].columns != hidden || w.matrices[2].columns != hidden ||
        w.head_norms[0].len != hw || w.head_norms[1].len != hw || w.matrices[0].rows % hw || w.matrices[1].rows % hw ||
        w.matrices[2].rows % hw || w.matrices[0].rows != w.attention.q_heads * hw ||
        w.matrices[1].rows != w.attention.kv_heads * hw || w.matrices[2].rows != w.matrices[1].rows ||
        w.attention.width != hw || w.output.columns != w.matrices[0].rows || w.output.rows != hidden ||
        f.gate.columns != hidden || f.up.columns != hidden || f.up.rows != f.gate.rows ||
        f.down.columns != f.gate.rows || f.down.rows != hidden || !std::isfinite(f.layer_scale))
        return fail(AF_ERR_INVALID, tag + ": incompatible consecutive-block dimensions or insufficient context");
    if ((rc = check_norm(w.input_norm, hidden, (tag + " input norm").c_str()))) return rc;
    if ((rc = check_norm(w.head_norms[0], hw, (tag + " q norm").c_str()))) return rc;
    if ((rc = check_norm(w.head_norms[1], hw, (tag + " k norm").c_str()))) return rc;
    if ((rc = check_norm(w.output_norm, hidden, (tag + " post-attention norm").c_str()))) return rc;
    if ((rc = check_norm(f.pre, hidden, (tag + " FFN norm").c_str()))) return rc;
    if ((rc = check_norm(f.post, hidden, (tag + " post-FFN norm").c_str()))) return rc;
    if ((rc = check_supported_attention(w.attention))) return rc;
    if ((rc = check_supported_q4(hidden, tag.c_str()))) return rc;
    if ((rc = check_supported_q4(f.gate.rows, tag.c_str()))) return rc;
    if ((rc = check_supported_q4(w.output.columns, tag.c_str()))) return rc;
    return AF_OK;
}

// K_LAYERS: plain launches of the step kernel; K_LAYERS_TL: launches that also write the in-kernel
// timeline (slower by the timestamp stores).
enum KernelKind { K_QKV = 0, K_ATTN, K_OPROJ, K_GATEUP, K_DOWN, K_HEAD, K_LAYERS, K_BARRIER, K_LAYERS_TL, K_KINDS };
const char* const kKindNames[K_KINDS] = {"qkv", "attention", "o_proj", "gate_up", "down", "head", "layers", "barrier",
                                         "layers_timeline"};

// Event pairs around individual launches (direct-launch profiling only).
struct KernelTimer {
    struct Rec {
        hipEvent_t a, b;
        int kind;
        double bytes;
    };
    std::vector<Rec> recs;
    size_t used = 0;
    ~KernelTimer() {
        for (auto& r : recs) {
            (void)hipEventDestroy(r.a);
            (void)hipEventDestroy(r.b);
        }
    }
    Rec* next() {
        if (used == recs.size()) {
            Rec r{};
            if (hipEventCreate(&r.a) != hipSuccess || hipEventCreate(&r.b) != hipSuccess) return nullptr;
            recs.push_back(r);
        }
        return &recs[used++];
    }
};

}  // namespace

struct af_session {
    std::vector<LayerDev> layers;
    Q6Dev head;
    DevMem final_norm;
    float final_eps = 0, emb_scale = 1, cap = 0;
    uint32_t hidden = 0, intermediate = 0, vocabulary = 0, capacity = 0;
    uint32_t max_qkv = 0, max_q = 0, cmax = 0, head_blocks = 0;
    DevMem X, H, QKV, ATT, PROJ, ACT, ACTIMG, D, QKVT, PROJT, DT, LOGITS, PART, COUNTERS, HPART, HCOUNT, STATE, IDS, STOPS,
        RESULT, SNAP, KVSNAP;
    // persistent step kernel: layer table, digit images, barrier words
    DevMem STEP_LAYERS, ATT_IMG, ACT_IMG, BAR, CLOCK, STREAM, STREAM_OFF, STREAM_RUNS;
    uint32_t clock_steps = 0, clock_used = 0;  // profiling: step timelines in CLOCK
    uint32_t clock_skip = 0;                     // profiling: plain launches before the timelines
    bool use_step = true;     // all layers of a step in one persistent launch
    uint32_t fail_phase = ~0u;  // AF_STEP_FAIL_PHASE: a step-kernel barrier that times out (tests)
    bool xcd_local = false;     // the step kernel's XCD-local layout (setup_step)
    bool attn_xl = false;       // attention launches' XCD-local merge (attn_xcd_local)
    uint32_t step_grid = 0, step_cmax = 0, group = 0;
    uint32_t step_attn_pre = 0, step_stage_clen = 0;  // an attention item's LDS (step_attn_layout)
    size_t step_lds = 0;
    // The step kernel takes runs of consecutive layers, one launch per run: a single run of every
    // layer, or, when some layers are outside its limits (Gemma 4's 512-wide global layers), the
    // runs between those, which the per-operation kernels take.  STEP_LAYERS holds the runs' layers
    // in order; STREAM_RUNS each run's byte range of every streaming wave's records.
    struct StepRun {
        uint32_t first, j0, n;  // first layer, its entry in STEP_LAYERS, layers
    };
    std::vector<StepRun> runs;
    std::vector<int32_t> run_at;   // per layer: the run starting there (-1: none)
    std::vector<uint8_t> in_step;  // per layer: 1 if a run holds it
    uint32_t step_q = 0, step_count = 0;  // the runs' query width and layers
    bool segmented() const { return runs.size() != 1 || runs[0].n != layers.size(); }
    uint32_t max_kv_rows = 0;
    StepRecord* records = nullptr;      // mapped host memory, capacity + 2 entries (host view)
    StepRecord* records_dev = nullptr;  // the same memory as the device addresses it
    uint32_t* state_host = nullptr;     // pinned staging for state uploads (read by the async copy)
    hipStream_t stream = nullptr;
    hipGraphExec_t decode_exec = nullptr, prefill_exec = nullptr;
    hipGraph_t decode_graph = nullptr, prefill_graph = nullptr;
    std::vector<hipEvent_t> events;
    hipEvent_t ev_start = nullptr;
    std::vector<uint32_t> cached;  // tokens of the conversation (GenerationSession prefix)
    uint32_t consumed = 0;         // positions with K/V in the caches
    bool poisoned = false;
    bool use_graphs = true;
    KernelTimer* timer = nullptr;  // set during af_session_profile
    // Batched prefill (batch.hip): prompt positions run through the layers up to kBatchMax at a time,
    // every weight read once per batch.  prefill_batch: positions per batch for generation
    // (AF_PREFILL_BATCH, default kBatchMax; 0 or 1 prefills one position per step-kernel launch);
    // trace_batch: the same for af_session_trace (AF_TRACE_BATCH, default 0: the step kernel).
    uint32_t prefill_batch = kBatchMax, trace_batch = 0;
    // Greedy speculative decoding with prompt-lookup drafts (AF_SPECULATIVE=1; AF_SPEC_DEPTH draft
    // tokens at most, default 11, at most kVerifyMax - 1): the draft and the pending token run through
    // the batched layers in one pass and the head checks the positions, up to four per launch.
    bool speculative = false;
    uint32_t spec_depth = 11;
    uint64_t spec_passes = 0, spec_drafted = 0, spec_accepted = 0;  // since open (af_session_speculation)
    uint32_t max_qh = 0, max_qh_part = 0;
    DevMem XB, HB, QKVB, QB, ATTB, PROJB, ACTB, DB, BIMG, BGEMM, BPART, BCOUNT;

    // Launches f(); when profiling, brackets it with an event pair tagged with its kind and bytes.
    template <typename F>
    hipError_t timed(int kind, double bytes, F f) {
        KernelTimer::Rec* r = timer ? timer->next() : nullptr;
        if (r) {
            r->kind = kind;
            r->bytes = bytes;
            hipError_t e = hipEventRecord(r->a, stream);
            if (e != hipSuccess) return e;
        }
        hipError_t e = f();
        if (e == hipSuccess && r) e = hipEventRecord(r->b, stream);
        return e;
    }
    static double q4_bytes(const Q4Dev& m) { return (double)m.rows * (m.columns / 32) * 18.0; }
    uint32_t host_pos = 0;  // position being consumed (profiling: attention bytes)

    ~af_session() {
        if (stream) (void)hipStreamSynchronize(stream);
        if (decode_exec) (void)hipGraphExecDestroy(decode_exec);
        if (prefill_exec) (void)hipGraphExecDestroy(prefill_exec);
        if (decode_graph) (void)hipGraphDestroy(decode_graph);
        if (prefill_graph) (void)hipGraphDestroy(prefill_graph);
        for (auto e : events) (void)hipEventDestroy(e);
        if (ev_start) (void)hipEventDestroy(ev_start);
        if (records) (void)hipHostFree(records);
        if (state_host) (void)hipHostFree(state_host);
        if (stream) (void)hipStreamDestroy(stream);
    }

    // One layer's five kernels.  Layer 0 embeds ids[pos]; later layers finish the
    // previous layer's FFN tail (post-norm, residual, scale) in their prologue.
    hipError_t enqueue_layer(uint32_t l, bool step) {
        LayerDev& L = layers[l];
        const uint32_t* st = step ? STATE.as<uint32_t>() : nullptr;
        Q4Args qa{};
        qa.w = L.qkv.view();
        qa.y = QKV.as<float>();
        qa.state = st;
        qa.in.w_n = L.input_norm.as<float>();
        qa.in.eps_n = L.input_eps;
        qa.in.x_out = X.as<float>();
        int kind;
        if (l == 0) {
            qa.in.table = head.view();
            qa.in.ids = IDS.as<uint32_t>();
            qa.in.state = STATE.as<uint32_t>();
            qa.in.emb_scale = emb_scale;
            kind = IN_EMBED;
        } else {
            const LayerDev& P = layers[l - 1];
            qa.in.x = D.as<float>();
            qa.in.res = H.as<float>();
            qa.in.w_a = P.post_ffn.as<float>();
            qa.in.eps_a = P.post_ffn_eps;
            qa.in.scale = P.layer_scale;
            kind = IN_RESID;
        }
        hipError_t e = timed(K_QKV, q4_bytes(L.qkv) + 4.0 * (3.0 * hidden + L.qkv.rows),
                             [&] { return launch_q4_gemv(qa, kind, OUT_PLAIN, L.qkv.rows, stream); });
        if (e != hipSuccess) return e;

        AttnArgs aa{};
        const float* qkv = QKV.as<float>();
        aa.q_raw = qkv;
        aa.k_raw = qkv + L.qn;
        aa.v_raw = L.shared_v ? qkv + L.qn : qkv + L.qn + L.kn;
        aa.q_norm = L.q_norm.as<float>();
        aa.k_norm = L.k_norm.as<float>();
        aa.q_eps = L.q_eps;
        aa.k_eps = L.k_eps;
        aa.v_eps = L.input_eps;
        aa.v_norm = L.v_norm;
        aa.inv_freq = L.inv_freq.as<double>();
        aa.kcache = L.kcache.as<uint16_t>();
        aa.vcache = L.vcache.as<uint16_t>();
        aa.ring = L.ring;
        aa.window = L.window;
        aa.scale = L.scale;
        aa.state = STATE.as<uint32_t>();
        aa.out = ATT.as<float>();
        aa.part = PART.as<float>();
        aa.counters = COUNTERS.as<uint32_t>();
        aa.cmax = cmax;
        aa.min_chunk = kAttnMinChunk;
        aa.kv_heads = L.kv_heads;
        aa.group = L.q_heads / L.kv_heads;
        aa.xcd_local = attn_xl ? 1u : 0u;
        const double nvis = L.window ? std::min<double>(host_pos + 1, L.window) : host_pos + 1.0;
        const double attn_bytes = nvis * 2.0 * L.kn * 2.0 + 4.0 * (2.0 * L.qn + 2.0 * L.kn) + 4.0 * L.kn;
        if ((e = timed(K_ATTN, attn_bytes, [&] { return launch_attention(aa, L.q_heads / L.kv_heads, L.width, stream); })) !=
            hipSuccess)
            return e;

        Q4Args oa{};
        oa.w = L.o.view();
        oa.in.x = ATT.as<float>();
        oa.y = PROJ.as<float>();
        oa.state = st;
        if ((e = timed(K_OPROJ, q4_bytes(L.o) + 4.0 * (L.qn + L.o.rows),
                       [&] { return launch_q4_gemv(oa, IN_PLAIN, OUT_PLAIN, L.o.rows, stream); })) != hipSuccess)
            return e;

        Q4Args ga{};
        ga.w = L.gate.view();
        ga.w2 = L.up.view();
        ga.in.x = PROJ.as<float>();
        ga.in.res = X.as<float>();
        ga.in.w_a = L.post_attn.as<float>();
        ga.in.eps_a = L.post_attn_eps;
        ga.in.scale = 1.0f;
        ga.in.w_n = L.ffn_norm.as<float>();
        ga.in.eps_n = L.ffn_eps;
        ga.in.x_out = H.as<float>();
        ga.y = ACT.as<float>();
        ga.dig_out = ACTIMG.as<int8_t>();  // the down GEMV's input, as its digit image
        ga.state = st;
        if ((e = timed(K_GATEUP, q4_bytes(L.gate) + q4_bytes(L.up) + 4.0 * (3.0 * hidden + intermediate),
                       [&] { return launch_q4_gemv(ga, IN_RESID, OUT_GELU, intermediate, stream); })) != hipSuccess)
            return e;

        Q4Args da{};
        da.w = L.down.view();
        da.in.dig = ACTIMG.as<int8_t>();
        da.y = D.as<float>();
        da.state = st;
        return timed(K_DOWN, q4_bytes(L.down) + 4.0 * (intermediate + hidden),
                     [&] { return launch_q4_gemv(da, IN_DIGITS, OUT_PLAIN, hidden, stream); });
    }

    HeadArgs head_args(bool step, bool with_logits) {
        const LayerDev& P = layers.back();
        HeadArgs h{};
        h.w = head.view();
        h.in.x = D.as<float>();
        h.in.res = H.as<float>();
        h.in.w_a = P.post_ffn.as<float>();
        h.in.eps_a = P.post_ffn_eps;
        h.in.scale = P.layer_scale;
        h.in.w_n = final_norm.as<float>();
        h.in.eps_n = final_eps;
        h.in.x_out = X.as<float>();
        h.logits = with_logits ? LOGITS.as<float>() : nullptr;
        h.partial = HPART.as<uint4>();
        h.counter = HCOUNT.as<uint32_t>();
        h.result = RESULT.as<uint32_t>();
        if (step) {
            h.state = STATE.as<uint32_t>();
            h.ids = IDS.as<uint32_t>();
            h.stop_ids = STOPS.as<uint32_t>();
            h.records = records_dev;
        }
        return h;
    }

    // Launch arguments of run k.  advance: the launch moves ST_POS on (a single run without the
    // head); the runs of a segmented step leave that to the end of the step.
    StepArgs step_args(uint32_t k, bool advance, float* snap) {
        const StepRun& r = runs[k];
        StepArgs a{};
        a.layers = STEP_LAYERS.as<StepLayer>() + r.j0;
        a.n_layers = r.n;
        a.hidden = hidden;
        a.inter = intermediate;
        a.table = head.view();
        a.emb_scale = emb_scale;
        a.ids = IDS.as<uint32_t>();
        a.state = STATE.as<uint32_t>();
        a.X = X.as<float>();
        a.H = H.as<float>();
        a.QKV = QKV.as<float>();
        a.PROJ = PROJ.as<float>();
        a.D = D.as<float>();
        a.QKVT = QKVT.as<uint32_t>();
        a.PROJT = PROJT.as<uint32_t>();
        a.DT = DT.as<uint32_t>();
        a.att_img = ATT_IMG.as<int8_t>();
        a.act_img = ACT_IMG.as<int8_t>();
        a.part = PART.as<float>();
        a.counters = COUNTERS.as<uint32_t>();
        a.bar = BAR.as<uint32_t>();
        a.stream = STREAM.as<uint8_t>();
        a.stream_off = STREAM_RUNS.as<uint64_t>() + (size_t)k * step_grid * kStepStreamWaves * 2;
        a.cmax = step_cmax;
        a.xs_off = step_xs_offset(hidden, intermediate, step_q);
        a.attn_pre_off = step_attn_pre;
        a.stage_clen = step_stage_clen;
        a.advance = advance ? 1u : 0u;
        a.snap = snap;
        a.fail_phase = k == 0 ? fail_phase : ~0u;
        a.xcd_local = xcd_local ? 1u : 0u;
        a.tag_stride = step_count;
        a.tag_base = r.j0;
        if (r.first > 0) {  // the layer before is the per-operation kernels'
            const LayerDev& P = layers[r.first - 1];
            a.prev_post_ffn = P.post_ffn.as<float>();
            a.prev_post_ffn_eps = P.post_ffn_eps;
            a.prev_scale = P.layer_scale;
        }
        return a;
    }

    uint32_t barriers() const { return 5 * (uint32_t)layers.size() - 1; }
    size_t clock_words() const { return (size_t)(barriers() + 1) * kStepMarks * step_grid; }

    // Weight bytes of run k's layers.
    double layer_bytes(uint32_t k = 0) const {
        double b = 0;
        for (uint32_t l = runs[k].first; l < runs[k].first + runs[k].n; ++l) {
            const LayerDev& L = layers[l];
            b += q4_bytes(L.qkv) + q4_bytes(L.o) + q4_bytes(L.gate) + q4_bytes(L.up) + q4_bytes(L.down);
        }
        return b;
    }

    // Every layer of a step, without the head or the position's advance: the step kernel's runs
    // and the per-operation kernels of the other layers, in layer order.
    hipError_t enqueue_layers() {
        for (uint32_t l = 0; l < layers.size();) {
            hipError_t e;
            if (use_step && in_step[l]) {
                const uint32_t k = (uint32_t)run_at[l];
                e = timed(K_LAYERS, layer_bytes(k),
                          [&] { return launch_step(step_args(k, false, nullptr), group, step_grid, step_lds, stream); });
                l += runs[k].n;
            } else {
                e = enqueue_layer(l, true);
                ++l;
            }
            if (e != hipSuccess) return e;
        }
        return hipSuccess;
    }

    hipError_t enqueue_step(bool with_head) {
        if (use_step && !segmented()) {
            StepArgs a = step_args(0, !with_head, nullptr);
            int kind = K_LAYERS;
            if (timer && clock_skip) {
                --clock_skip;
            } else if (timer && clock_used < clock_steps) {
                a.clock = CLOCK.as<uint64_t>() + (size_t)clock_used++ * clock_words();
                hipError_t e = hipMemsetAsync(a.clock, 0, clock_words() * 8, stream);  // profiling only
                if (e != hipSuccess) return e;
                kind = K_LAYERS_TL;
            }
            hipError_t e = timed(kind, layer_bytes(), [&] { return launch_step(a, group, step_grid, step_lds, stream); });
            if (e != hipSuccess || !with_head) return e;
            return timed(K_HEAD, (double)head.rows * (head.columns / 256) * 210.0 + 4.0 * 3.0 * hidden,
                         [&] { return launch_head(head_args(true, false), IN_RESID, head_blocks, stream); });
        }
        hipError_t e = enqueue_layers();
        if (e != hipSuccess) return e;
        if (with_head)
            return timed(K_HEAD, (double)head.rows * (head.columns / 256) * 210.0 + 4.0 * 3.0 * hidden,
                         [&] { return launch_head(head_args(true, false), IN_RESID, head_blocks, stream); });
        return launch_advance(STATE.as<uint32_t>(), stream);
    }

    int capture(bool with_head, hipGraph_t& g, hipGraphExec_t& x) {
        HIP_OK(hipStreamBeginCapture(stream, hipStreamCaptureModeThreadLocal), "graph capture begin");
        hipError_t e = enqueue_step(with_head);
        hipError_t e2 = hipStreamEndCapture(stream, &g);
        HIP_OK(e, "graph capture");
        HIP_OK(e2, "graph capture end");
        HIP_OK(hipGraphInstantiate(&x, g, nullptr, nullptr, 0), "graph instantiate");
        HIP_OK(hipGraphUpload(x, stream), "graph upload");
        return AF_OK;
    }

    // One decode (with_head) or prefill step: a replay of the graph captured at open, or direct
    // launches (AF_DISABLE_GRAPHS).  Every argument of a step's launches is fixed for the session
    // (the position, ids and stop state live in device memory), so one graph serves every token.
    hipError_t run_step(bool with_head) {
        if (use_graphs) return hipGraphLaunch(with_head ? decode_exec : prefill_exec, stream);
        return enqueue_step(with_head);
    }

    // The staging words are only rewritten after the stream has drained (every caller
    // synchronises before returning), so the async copy never reads a changed value.
    int set_state(uint32_t pos, uint32_t nstop) {
        state_host[ST_POS] = pos;
        state_host[ST_BAD] = 0u;
        state_host[ST_STOP] = 0u;
        state_host[ST_NSTOP] = nstop;
        HIP_OK(hipMemcpyAsync(STATE.p, state_host, ST_HOST_WORDS * 4, hipMemcpyHostToDevice, stream), "state upload");
        return AF_OK;
    }

    // After the stream has drained: true if a step-kernel launch timed out in a grid barrier or a
    // tagged poll (state word ST_BAD = 2; the failed step's position is left in ST_POS).
    int step_timed_out(bool& out, uint32_t* pos) {
        out = false;
        if (!use_step) return AF_OK;
        uint32_t words[ST_WORDS] = {};
        HIP_OK(hipMemcpy(words, STATE.p, sizeof(words), hipMemcpyDeviceToHost), "state download");
        out = words[ST_BAD] == 2u;
        if (pos) *pos = words[ST_POS];
        return AF_OK;
    }

    // The persistent step kernel needs every workgroup of its grid resident at once; when they
    // were not (its barrier or a tagged poll timed out), the session continues on the
    // per-operation kernels, which make no such assumption.  The failed step is run again there by
    // the caller: a step recomputes its activations from the embedding, and the K/V slots a failed
    // step wrote are its own position's, which the rerun overwrites.  The attention merge tickets
    // an interrupted merge left are cleared; the graphs are recaptured for the new path.
    int fall_back() {
        use_step = false;
        HIP_OK(hipMemsetAsync(COUNTERS.p, 0, COUNTERS.bytes, stream), "attention counters clear");
        HIP_OK(hipStreamSynchronize(stream), "fall-back");
        if (use_graphs) {
            if (decode_exec) (void)hipGraphExecDestroy(decode_exec);
            if (prefill_exec) (void)hipGraphExecDestroy(prefill_exec);
            if (decode_graph) (void)hipGraphDestroy(decode_graph);
            if (prefill_graph) (void)hipGraphDestroy(prefill_graph);
            decode_exec = prefill_exec = nullptr;
            decode_graph = prefill_graph = nullptr;
            int rc = capture(true, decode_graph, decode_exec);
            if (rc) return rc;
            if ((rc = capture(false, prefill_graph, prefill_exec))) return rc;
        }
        return AF_OK;
    }


    int ensure_batch() {
        if (XB.p) return AF_OK;
        uint32_t blocks = std::max({hidden, max_q, intermediate}) / 32;
        size_t part = 4;
        for (const LayerDev& L : layers) {
            part = std::max({part, batch_gemm_part_bytes(L.qkv.rows, hidden / 32, kBatchMax, false),
                             batch_gemm_part_bytes(L.o.rows, L.qn / 32, kBatchMax, false),
                             batch_gemm_part_bytes(L.gate.rows, hidden / 32, kBatchMax, true),
                             batch_gemm_part_bytes(L.down.rows, intermediate / 32, kBatchMax, false)});
        }
        const size_t T = kBatchMax;
        struct {
            DevMem* m;
            size_t bytes;
        } bufs[] = {
            {&XB, T * hidden * 4},        {&HB, T * hidden * 4},  {&QKVB, T * max_qkv * 4},
            {&ATTB, T * max_q * 4},       {&QB, T * max_q * 4},   {&PROJB, T * hidden * 4},
            {&ACTB, T * intermediate * 4},
            {&DB, T * hidden * 4},        {&BIMG, batch_image_bytes(blocks, kBatchMax)}, {&BGEMM, part},
            {&BPART, T * kBatchAttnChunks * max_qh_part * 4}, {&BCOUNT, T * std::max<uint32_t>(max_qh, 64) * 4},
        };
        for (auto& b : bufs) {
            int rc = dev_alloc(*b.m, b.bytes, "batch buffer");
            if (rc) return rc;
        }
        HIP_OK(hipMemsetAsync(BCOUNT.p, 0, BCOUNT.bytes, stream), "batch counters clear");
        return AF_OK;
    }

    // Digit image of T vectors for the GEMV of matrix m (see BatchIn).
    BatchIn batch_in(int mode, uint32_t T, uint32_t K, const float* x, size_t stride) {
        BatchIn in{};
        in.mode = mode;
        in.T = T;
        in.K = K;
        in.stride = stride;
        in.x = x;
        in.scale = 1.0f;
        in.img = BIMG.as<int8_t>();
        return in;
    }

    // parts non-null: the split-K partials may stay in BGEMM for the next input kernel, which then
    // sums them; *parts tells it how many (0: y written).
    hipError_t batch_gemm(const Q4Dev& m, const Q4Dev* m2, uint32_t T, float* y, size_t y_stride,
                          uint32_t* parts = nullptr) {
        BatchGemm g{};
        g.w = m.view();
        if (m2) g.w2 = m2->view();
        g.img = BIMG.as<int8_t>();
        g.T = T;
        g.y = y;
        g.y_stride = y_stride;
        g.part = BGEMM.as<float>();
        g.defer = parts != nullptr;
        return launch_batch_gemm(g, m2 != nullptr, stream, parts);
    }

    // A BI_RESID input whose x is the output y of the GEMM before it: the GEMM's partials when it
    // deferred its reduce (parts > 0), else y.
    BatchIn resid_input(uint32_t T, const float* y, uint32_t parts) {
        BatchIn in = batch_in(BI_RESID, T, hidden, y, hidden);
        if (parts) {
            in.part = BGEMM.as<float>();
            in.parts = parts;
            in.part_row = (size_t)(hidden + 15) / 16 * 16;
        }
        return in;
    }

    // Runs positions p0 .. p0 + T - 1 (ids in IDS) through every layer, appending their K/V; leaves
    // the last layer's down output in DB and FFN residual in HB.  snap: layer outputs [T][layers][hidden]
    // (null: none).  The decoder layer as the step kernel computes it (crates/cuda-backend/src/stack.rs
    // 502-700, run_batch), with the GEMVs over the batch.
    hipError_t enqueue_batch(uint32_t p0, uint32_t T, float* snap) {
        const size_t H = hidden, nl = layers.size();
        hipError_t e;
        uint32_t down_parts = 0;  // the previous layer's down partials left in BGEMM
        for (uint32_t l = 0; l < nl; ++l) {
            LayerDev& L = layers[l];
            BatchIn in = l == 0 ? batch_in(BI_EMBED, T, hidden, nullptr, H) : resid_input(T, DB.as<float>(), down_parts);
            in.w_n = L.input_norm.as<float>();
            in.eps_n = L.input_eps;
            in.x_out = XB.as<float>();
            if (l == 0) {
                in.table = head.view();
                in.ids = IDS.as<uint32_t>();
                in.pos0 = p0;
                in.emb_scale = emb_scale;
            } else {
                const LayerDev& P = layers[l - 1];
                in.res = HB.as<float>();
                in.w_a = P.post_ffn.as<float>();
                in.eps_a = P.post_ffn_eps;
                in.scale = P.layer_scale;
                if (snap) {
                    in.snap = snap + (l - 1) * H;
                    in.snap_stride = nl * H;
                }
            }
            if ((e = launch_batch_input(in, stream)) != hipSuccess) return e;
            uint32_t qkv_parts = 0;  // the append pass sums qkv's partials when its reduce is deferred
            if ((e = batch_gemm(L.qkv, nullptr, T, QKVB.as<float>(), L.qkv.rows, &qkv_parts)) != hipSuccess) return e;

            AttnArgs aa{};
            const float* qkv = QKVB.as<float>();
            aa.q_raw = qkv;
            aa.k_raw = qkv + L.qn;
            aa.v_raw = L.shared_v ? qkv + L.qn : qkv + L.qn + L.kn;
            aa.in_stride = L.qkv.rows;
            aa.q_norm = L.q_norm.as<float>();
            aa.k_norm = L.k_norm.as<float>();
            aa.q_eps = L.q_eps;
            aa.k_eps = L.k_eps;
            aa.v_eps = L.input_eps;
            aa.v_norm = L.v_norm;
            aa.inv_freq = L.inv_freq.as<double>();
            aa.kcache = L.kcache.as<uint16_t>();
            aa.vcache = L.vcache.as<uint16_t>();
            aa.ring = L.ring;
            aa.window = L.window;
            aa.scale = L.scale;
            aa.position = p0;
            aa.out = ATTB.as<float>();
            aa.out_stride = L.qn;
            aa.part = BPART.as<float>();
            aa.counters = BCOUNT.as<uint32_t>();
            aa.cmax = 1;  // the append pass: one block per (token, KV head, query group)
            aa.min_chunk = kAttnMinChunk;
            aa.kv_heads = L.kv_heads;
            aa.group = L.q_heads / L.kv_heads;
            aa.mode = ATT_APPEND;
            aa.q_out = QB.as<float>();
            if (qkv_parts) {
                aa.raw_part = BGEMM.as<float>();
                aa.raw_parts = qkv_parts;
                aa.raw_prow = (L.qkv.rows + 15) / 16 * 16;
                aa.raw_tp = (T + 15) / 16 * 16;
            }
            if ((e = launch_attention(aa, aa.group, L.width, stream, T)) != hipSuccess) return e;
            BatchAttn ba{};
            ba.q = QB.as<float>();
            ba.kcache = L.kcache.as<uint16_t>();
            ba.vcache = L.vcache.as<uint16_t>();
            ba.ring = L.ring;
            ba.window = L.window;
            ba.T = T;
            ba.pos0 = p0;
            ba.kv_heads = L.kv_heads;
            ba.group = L.q_heads / L.kv_heads;
            ba.scale = L.scale;
            ba.part = BPART.as<float>();
            ba.out = ATTB.as<float>();
            ba.out_stride = L.qn;
            if ((e = launch_batch_attention(ba, L.width, stream)) != hipSuccess) return e;

            in = batch_in(BI_PLAIN, T, L.qn, ATTB.as<float>(), L.qn);
            if ((e = launch_batch_input(in, stream)) != hipSuccess) return e;
            uint32_t o_parts = 0;
            if ((e = batch_gemm(L.o, nullptr, T, PROJB.as<float>(), H, &o_parts)) != hipSuccess) return e;

            in = resid_input(T, PROJB.as<float>(), o_parts);
            in.res = XB.as<float>();
            in.w_a = L.post_attn.as<float>();
            in.eps_a = L.post_attn_eps;
            in.w_n = L.ffn_norm.as<float>();
            in.eps_n = L.ffn_eps;
            in.x_out = HB.as<float>();
            if ((e = launch_batch_input(in, stream)) != hipSuccess) return e;
            uint32_t ff_parts = 0;
            if ((e = batch_gemm(L.gate, &L.up, T, ACTB.as<float>(), intermediate, &ff_parts)) != hipSuccess) return e;

            in = batch_in(BI_PLAIN, T, intermediate, ACTB.as<float>(), intermediate);
            if (ff_parts) {
                in.part = BGEMM.as<float>();
                in.parts = ff_parts;
                in.part_row = (size_t)(intermediate + 15) / 16 * 16;
            }
            if ((e = launch_batch_input(in, stream)) != hipSuccess) return e;
            // the last layer's down output stays in DB for the caller
            if ((e = batch_gemm(L.down, nullptr, T, DB.as<float>(), H, l + 1 < nl ? &down_parts : nullptr)) !=
                hipSuccess)
                return e;
        }
        if (!snap) return hipSuccess;
        // the last layer's output (its image is not used)
        const LayerDev& P = layers.back();
        BatchIn in = batch_in(BI_RESID, T, hidden, DB.as<float>(), H);
        in.res = HB.as<float>();
        in.w_a = P.post_ffn.as<float>();
        in.eps_a = P.post_ffn_eps;
        in.scale = P.layer_scale;
        in.x_out = XB.as<float>();
        in.snap = snap + (nl - 1) * H;
        in.snap_stride = nl * H;
        return launch_batch_input(in, stream);
    }

    // Positions [from, to) through the batched layers (K/V appended), in batches of `batch`.
    hipError_t prefill_batched(uint32_t from, uint32_t to, uint32_t batch) {
        for (uint32_t p = from; p < to; p += batch) {
            hipError_t e = enqueue_batch(p, std::min(batch, to - p), nullptr);
            if (e != hipSuccess) return e;
        }
        return hipSuccess;
    }
};

namespace {

// Prepares the persistent step kernel: one launch of one workgroup per CU runs a run of layers
// (every layer when all are within its limits).  Its layers share the attention geometry of the
// first 256-wide layer (query group, query width); a layer outside its limits (another geometry,
// GEMV rows beyond two units per workgroup, attention chunks beyond its LDS) runs on the
// per-operation kernels between two runs, and then every step layer must have the first one's
// shapes, so that each streaming wave holds the same records per layer.  A model with no such
// layer keeps the per-operation kernels in a graph.
int setup_step(af_session& s) {
    if (!s.use_step) return AF_OK;
    const uint32_t nl = (uint32_t)s.layers.size();
    const LayerDev* R = nullptr;
    for (const LayerDev& L : s.layers)
        if (L.width == 256) {
            R = &L;
            break;
        }
    if (!R) {
        s.use_step = false;
        return AF_OK;
    }
    const uint32_t group = R->q_heads / R->kv_heads, step_q = R->qn;
    const size_t lds = step_lds_bytes(s.hidden, s.intermediate, step_q, group);
    uint32_t grid = 0;
    HIP_OK(step_max_grid(group, lds, &grid), "step kernel occupancy");
    bool fits = grid >= 8 && s.hidden <= 4096 && s.hidden % 32 == 0;
    const auto geometry = [&](const LayerDev& L) {
        return L.width == 256 && L.q_heads / L.kv_heads == group && L.o.columns == step_q;
    };
    uint32_t kv_max = 1;
    for (const LayerDev& L : s.layers)
        if (geometry(L)) kv_max = std::max(kv_max, L.kv_heads);
    const uint32_t cm = std::min(grid / kv_max, step_merge_chunks(group, lds));
    fits = fits && cm >= 1 && cm <= kStepMaxChunks;
    s.in_step.assign(nl, 0);
    uint32_t count = 0;
    for (uint32_t i = 0; i < nl && fits; ++i) {
        const LayerDev& L = s.layers[i];
        const uint32_t span = L.window ? std::min(L.window, s.capacity) : s.capacity;
        if (geometry(L) && (span + cm - 1) / cm <= kStepMaxClen && (L.qkv.rows + 15) / 16 <= kStepMaxUnits * grid &&
            (L.o.rows + 15) / 16 <= kStepMaxUnits * grid && (s.intermediate + 31) / 32 <= kStepMaxUnits * grid &&
            (L.down.rows + 15) / 16 <= kStepMaxUnits * grid) {
            s.in_step[i] = 1;
            ++count;
        }
    }
    if (count < nl)
        for (uint32_t i = 0; i < nl; ++i) {
            const LayerDev& L = s.layers[i];
            if (s.in_step[i] && !(L.q_heads == R->q_heads && L.kv_heads == R->kv_heads && L.shared_v == R->shared_v &&
                                  L.qkv.rows == R->qkv.rows && L.o.rows == R->o.rows))
                fits = false;
        }
    if (!fits || count == 0) {
        s.use_step = false;
        return AF_OK;
    }
    s.runs.clear();
    s.run_at.assign(nl, -1);
    for (uint32_t i = 0, j = 0; i < nl;) {
        if (!s.in_step[i]) {
            ++i;
            continue;
        }
        af_session::StepRun r{i, j, 0};
        for (; i < nl && s.in_step[i]; ++i, ++j) ++r.n;
        s.run_at[r.first] = (int32_t)s.runs.size();
        s.runs.push_back(r);
    }
    s.step_grid = grid;
    s.step_cmax = cm;
    step_attn_layout(s.hidden, s.intermediate, step_q, group, &s.step_attn_pre, &s.step_stage_clen);
    s.group = group;
    s.step_lds = lds;
    s.step_q = step_q;
    s.step_count = count;
    int rc;
    // XCD-local layout (StepArgs::xcd_local): BASELINE's attention geometry (8 KV heads of two query
    // heads, width 256, separate V) on a 256-workgroup grid whose workgroups b and b + 8 share an XCD
    // (workgroup b on XCD (x0 + b) % 8, where x0 varies from launch to launch), which a probe launch
    // checks on this device; AF_STEP_XCD_LOCAL=0 turns it off.
    bool xl = grid == 256 && group == 2 && !(std::getenv("AF_STEP_XCD_LOCAL") &&
                                              std::strcmp(std::getenv("AF_STEP_XCD_LOCAL"), "0") == 0);
    for (uint32_t i = 0; i < nl; ++i) {
        const LayerDev& L = s.layers[i];
        xl = xl && (!s.in_step[i] || (L.kv_heads == kXcds && L.q_heads == 2 * kXcds && L.width == 256 && !L.shared_v &&
                                      L.qkv.rows == (L.q_heads + 2 * L.kv_heads) * 256u));
    }
    if (xl) {
        DevMem map;
        if ((rc = dev_alloc(map, (size_t)grid * 4, "XCD map"))) return rc;
        HIP_OK(step_xcd_map(grid, map.as<uint32_t>(), nullptr), "XCD map");
        std::vector<uint32_t> xcc(grid);
        HIP_OK(hipMemcpy(xcc.data(), map.p, (size_t)grid * 4, hipMemcpyDeviceToHost), "XCD map");
        for (uint32_t b = 0; b < grid; ++b) xl = xl && xcc[b] == (xcc[0] + b) % kXcds;
    }
    s.xcd_local = xl;
    std::vector<StepLayer> table;
    for (uint32_t i = 0; i < nl; ++i) {
        if (!s.in_step[i]) continue;
        const LayerDev& L = s.layers[i];
        StepLayer& t = table.emplace_back();
        t.qkv = L.qkv.view();
        t.o = L.o.view();
        t.gate = L.gate.view();
        t.up = L.up.view();
        t.down = L.down.view();
        t.input_norm = L.input_norm.as<float>();
        t.q_norm = L.q_norm.as<float>();
        t.k_norm = L.k_norm.as<float>();
        t.post_attn = L.post_attn.as<float>();
        t.ffn_norm = L.ffn_norm.as<float>();
        t.post_ffn = L.post_ffn.as<float>();
        t.inv_freq = L.inv_freq.as<double>();
        t.kcache = L.kcache.as<uint16_t>();
        t.vcache = L.vcache.as<uint16_t>();
        t.input_eps = L.input_eps;
        t.q_eps = L.q_eps;
        t.k_eps = L.k_eps;
        t.v_eps = L.input_eps;
        t.post_attn_eps = L.post_attn_eps;
        t.ffn_eps = L.ffn_eps;
        t.post_ffn_eps = L.post_ffn_eps;
        t.layer_scale = L.layer_scale;
        t.scale = L.scale;
        t.q_heads = L.q_heads;
        t.kv_heads = L.kv_heads;
        t.qn = L.qn;
        t.kn = L.kn;
        t.v_off = L.shared_v ? L.qn : L.qn + L.kn;
        t.ring = L.ring;
        t.window = L.window;
        t.v_norm = L.v_norm ? 1u : 0u;
        t.chunks_max =
            L.window && L.window <= kStepWindowChunks * s.step_stage_clen ? std::min(cm, kStepWindowChunks) : cm;
    }
    if ((rc = dev_upload(s.STEP_LAYERS, table.data(), table.size() * sizeof(StepLayer), "layer table"))) return rc;
    // the o-proj input image is handed over as tagged pieces: 16 bytes per 8-byte image word
    const size_t att_img = (size_t)((s.max_q / 32 + 3) / 4) * kStepImg * 2,
                 act_img = (size_t)((s.intermediate / 32 + 3) / 4) * kStepImg;
    if ((rc = dev_alloc(s.ATT_IMG, att_img, "digit image"))) return rc;
    if ((rc = dev_alloc(s.ACT_IMG, act_img, "digit image"))) return rc;
    if ((rc = dev_alloc(s.BAR, kStepBarBytes, "barrier words"))) return rc;
    HIP_OK(hipMemset(s.ATT_IMG.p, 0, att_img), "digit image clear");
    HIP_OK(hipMemset(s.ACT_IMG.p, 0, act_img), "digit image clear");
    HIP_OK(hipMemset(s.BAR.p, 0, kStepBarBytes), "barrier clear");
    const size_t part = (size_t)grid * step_part_stride(group) * 4;
    if (s.PART.bytes < part) {
        if ((rc = dev_alloc(s.PART, part, "attention partials"))) return rc;
    }
    // The weight stream: each streaming wave's records, every phase of every layer in order, built
    // on the device from the tiled matrices, which the step kernel then no longer needs.
    const uint32_t nw = grid * kStepStreamWaves;
    std::vector<uint64_t> off((size_t)nw + 1, 0);
    for (uint32_t i = 0; i < nw; ++i) {
        const uint32_t b = i / kStepStreamWaves, w = i % kStepStreamWaves + 1;
        uint64_t recs = 0;
        for (uint32_t li = 0; li < nl; ++li) {
            if (!s.in_step[li]) continue;
            const LayerDev& L = s.layers[li];
            recs += step_wave_records((L.qkv.rows + 15) / 16, 1, (L.qkv.columns / 32 + 3) / 4, b, grid, w);
            recs += step_wave_records((L.o.rows + 15) / 16, 1, (L.o.columns / 32 + 3) / 4, b, grid, w);
            recs += step_wave_records((L.gate.rows + 31) / 32, 4, (L.gate.columns / 32 + 3) / 4, b, grid, w);
            recs += step_wave_records((L.down.rows + 15) / 16, 1, (L.down.columns / 32 + 3) / 4, b, grid, w);
        }
        off[i + 1] = off[i] + recs * kStepRecord;
    }
    if ((rc = dev_upload(s.STREAM_OFF, off.data(), off.size() * 8, "weight stream offsets"))) return rc;
    // each run's range of every wave's records (the runs' layers have equal shapes when there are
    // several, so a wave holds (off[i + 1] - off[i]) / count bytes per layer)
    std::vector<uint64_t> ranges(s.runs.size() * nw * 2);
    for (size_t k = 0; k < s.runs.size(); ++k)
        for (uint32_t i = 0; i < nw; ++i) {
            const uint64_t per = (off[i + 1] - off[i]) / count;
            ranges[(k * nw + i) * 2] = off[i] + s.runs[k].j0 * per;
            ranges[(k * nw + i) * 2 + 1] = s.runs.size() == 1 ? off[i + 1] : off[i] + (s.runs[k].j0 + s.runs[k].n) * per;
        }
    if ((rc = dev_upload(s.STREAM_RUNS, ranges.data(), ranges.size() * 8, "weight stream ranges"))) return rc;
    if ((rc = dev_alloc(s.STREAM, off.back() + kStepStreamPad, "weight stream"))) return rc;
    HIP_OK(hipMemset(s.STREAM.as<uint8_t>() + off.back(), 0, kStepStreamPad), "weight stream padding");
    HIP_OK(launch_stream_repack(s.STEP_LAYERS.as<StepLayer>(), count, grid, s.xcd_local ? 1u : 0u,
                                s.STREAM.as<uint8_t>(), s.STREAM_OFF.as<uint64_t>(), nullptr),
           "weight stream build");
    HIP_OK(hipDeviceSynchronize(), "weight stream build");
    // The tiled matrices stay resident: a step kernel that times out (its workgroups were not all
    // resident at once) makes the session fall back to the per-operation kernels, which read them.
    return AF_OK;
}

int open_session(const af_layer_weights* layers, uint32_t n_layers, const af_output_head* head, uint32_t capacity,
                 af_session** out) {
    if (!out) return fail(AF_ERR_INVALID, "null output");
    *out = nullptr;
    if (!layers || !head || n_layers == 0 || n_layers > 256 || capacity == 0 || capacity > AF_MAX_CONTEXT)
        return fail(AF_ERR_INVALID, "session limited to 1..256 blocks and " + std::to_string(AF_MAX_CONTEXT) +
                                        " tokens of context");
    int rc;
    const af_matrix& hm = head->matrix;
    if ((rc = check_q6(hm.bytes, hm.len, hm.columns, hm.rows, "output head"))) return rc;
    const uint32_t hidden = hm.columns;
    if (hidden > 4096) return fail(AF_ERR_INVALID, "hidden width above 4096 is not supported by the head");
    if ((rc = check_norm(head->norm, hidden, "output norm"))) return rc;
    if (!std::isfinite(head->cap) || head->cap <= 0.0f) return fail(AF_ERR_INVALID, "incompatible output head");
    const uint32_t inter = layers[0].ffn.gate.rows;
    for (uint32_t i = 0; i < n_layers; ++i) {
        if ((rc = validate_layer(layers[i], hidden, capacity, i))) return rc;
        if (layers[i].ffn.gate.rows != inter) return fail(AF_ERR_INVALID, "FFN width differs across layers");
    }
    if ((rc = ensure_device())) return rc;

    auto s = std::make_unique<af_session>();
    s->hidden = hidden;
    s->intermediate = inter;
    s->vocabulary = hm.rows;
    s->capacity = capacity;
    s->final_eps = head->norm.epsilon;
    s->cap = head->cap;
    s->emb_scale = std::sqrt((float)hidden);  // EmbeddingBatch::scale (crates/domain/src/embedding.rs:49-51)
    const char* env = std::getenv("AF_DISABLE_GRAPHS");
    s->use_graphs = !(env && *env && std::strcmp(env, "0") != 0);
    const char* step_env = std::getenv("AF_STEP_KERNEL");
    s->use_step = !(step_env && std::strcmp(step_env, "0") == 0);
    // A test of the fall-back path: the step kernel's barrier opening this phase (5 l + 4 opens
    // layer l's down projection) waits for one arrival more than the grid makes, and times out.
    if (const char* fp = std::getenv("AF_STEP_FAIL_PHASE")) s->fail_phase = (uint32_t)std::strtoul(fp, nullptr, 10);
    if (const char* pb = std::getenv("AF_PREFILL_BATCH"))
        s->prefill_batch = std::min<uint32_t>((uint32_t)std::strtoul(pb, nullptr, 10), kBatchMax);
    if (const char* tb = std::getenv("AF_TRACE_BATCH"))
        s->trace_batch = std::min<uint32_t>((uint32_t)std::strtoul(tb, nullptr, 10), kBatchMax);
    if (const char* sp = std::getenv("AF_SPECULATIVE")) s->speculative = std::strcmp(sp, "1") == 0;
    if (const char* sd = std::getenv("AF_SPEC_DEPTH"))
        s->spec_depth = std::max<uint32_t>(1, std::min<uint32_t>((uint32_t)std::strtoul(sd, nullptr, 10), kVerifyMax - 1));
    HIP_OK(hipStreamCreateWithFlags(&s->stream, hipStreamNonBlocking), "session stream");

    uint32_t max_kv = 0, max_q = 0, max_group = 1, max_qh_part = 0, max_qh = 0;
    s->layers.resize(n_layers);
    for (uint32_t i = 0; i < n_layers; ++i) {
        const af_layer_weights& w = layers[i];
        LayerDev& L = s->layers[i];
        L.q_heads = w.attention.q_heads;
        L.kv_heads = w.attention.kv_heads;
        L.width = w.attention.width;
        L.window = w.attention.window;
        L.scale = w.attention.scale;
        L.qn = w.matrices[0].rows;
        L.kn = w.matrices[1].rows;
        L.shared_v = w.matrices[2].bytes == w.matrices[1].bytes;
        L.v_norm = (w.flags & AF_LAYER_V_NORM) != 0;
        L.input_eps = w.input_norm.epsilon;
        L.q_eps = w.head_norms[0].epsilon;
        L.k_eps = w.head_norms[1].epsilon;
        L.post_attn_eps = w.output_norm.epsilon;
        L.ffn_eps = w.ffn.pre.epsilon;
        L.post_ffn_eps = w.ffn.post.epsilon;
        L.layer_scale = w.ffn.layer_scale;
        std::vector<af_matrix> qkv = {w.matrices[0], w.matrices[1]};
        if (!L.shared_v) qkv.push_back(w.matrices[2]);
        if ((rc = upload_q4(L.qkv, qkv))) return rc;
        if ((rc = upload_q4(L.o, {w.output}))) return rc;
        if ((rc = upload_q4(L.gate, {w.ffn.gate}))) return rc;
        if ((rc = upload_q4(L.up, {w.ffn.up}))) return rc;
        if ((rc = upload_q4(L.down, {w.ffn.down}))) return rc;
        if ((rc = dev_upload(L.input_norm, w.input_norm.weights, (size_t)hidden * 4, "norm upload"))) return rc;
        if ((rc = dev_upload(L.q_norm, w.head_norms[0].weights, (size_t)L.width * 4, "norm upload"))) return rc;
        if ((rc = dev_upload(L.k_norm, w.head_norms[1].weights, (size_t)L.width * 4, "norm upload"))) return rc;
        if ((rc = dev_upload(L.post_attn, w.output_norm.weights, (size_t)hidden * 4, "norm upload"))) return rc;
        if ((rc = dev_upload(L.ffn_norm, w.ffn.pre.weights, (size_t)hidden * 4, "norm upload"))) return rc;
        if ((rc = dev_upload(L.post_ffn, w.ffn.post.weights, (size_t)hidden * 4, "norm upload"))) return rc;
        std::vector<double> f = inverse_frequencies(w.rope);
        if ((rc = dev_upload(L.inv_freq, f.data(), f.size() * 8, "RoPE upload"))) return rc;
        // Sliding-window layers keep a ring of window + kBatchMax slots (crates/cuda-backend/src/
        // stack.rs:94-102): a batch appends up to kBatchMax positions before any of them attends,
        // and the first still sees its window - 1 predecessors.
        L.ring = L.window ? std::min(L.window + kBatchMax, capacity) : capacity;
        const size_t kv = (size_t)L.kv_heads * L.ring * L.width * 2;
        if ((rc = dev_alloc(L.kcache, kv, "K cache"))) return rc;
        if ((rc = dev_alloc(L.vcache, kv, "V cache"))) return rc;
        HIP_OK(hipMemset(L.kcache.p, 0, kv), "K cache clear");
        HIP_OK(hipMemset(L.vcache.p, 0, kv), "V cache clear");
        max_kv = std::max(max_kv, L.kv_heads);
        max_q = std::max(max_q, L.qn);
        max_group = std::max(max_group, L.q_heads / L.kv_heads);
        // per chunk: attention_kernel's partials (attn_part_row), at least the batched attention's (width + 2)
        max_qh_part = std::max(max_qh_part, L.q_heads * attn_part_row(L.width));
        max_qh = std::max(max_qh, L.q_heads);
        s->max_qkv = std::max(s->max_qkv, L.qkv.rows);
        s->max_kv_rows = std::max(s->max_kv_rows, L.kn);
    }
    s->max_q = max_q;
    s->max_qh = max_qh;
    s->max_qh_part = max_qh_part;
    if ((rc = upload_q6(s->head, hm.bytes, hm.columns, hm.rows))) return rc;
    if ((rc = dev_upload(s->final_norm, head->norm.weights, (size_t)hidden * 4, "final norm"))) return rc;

    s->cmax = kAttnMaxChunks;  // capacity <= AF_MAX_CONTEXT <= kAttnMaxChunks * kAttnMaxChunkLen
    s->head_blocks = head_grid(hm.rows);
    struct {
        DevMem* m;
        size_t bytes;
        bool zero;
    } bufs[] = {
        {&s->X, (size_t)hidden * 4, true},
        {&s->H, (size_t)hidden * 4, true},
        {&s->QKV, (size_t)s->max_qkv * 4, true},
        {&s->ATT, (size_t)max_q * 4, true},
        {&s->PROJ, (size_t)hidden * 4, true},
        {&s->ACT, (size_t)inter * 4, true},
        {&s->ACTIMG, (size_t)(inter + 127) / 128 * kStepImg, true},  // the down GEMV's input digit image
        {&s->D, (size_t)hidden * 4, true},
        {&s->QKVT, (size_t)s->max_qkv * 8, true},  // (value, tag) pairs: tag 0 is never current
        {&s->PROJT, (size_t)hidden * 8, true},
        {&s->DT, (size_t)hidden * 8, true},
        {&s->LOGITS, (size_t)hm.rows * 4, false},
        {&s->PART, (size_t)s->cmax * std::max<uint32_t>(max_qh_part, max_kv * step_part_stride(max_group)) * 4, false},
        {&s->COUNTERS, (size_t)std::max<uint32_t>(max_qh, 64) * 4, true},
        {&s->HPART, (size_t)s->head_blocks * 16 * kHeadBatchMax, false},  // (the verification head's per vector)
        {&s->HCOUNT, 256, true},
        {&s->STATE, ST_WORDS * 4, true},
        {&s->IDS, ((size_t)capacity + 2) * 4, true},
        {&s->STOPS, kMaxStopIds * 4, true},
        {&s->RESULT, 256, true},
    };
    for (auto& b : bufs) {
        if ((rc = dev_alloc(*b.m, b.bytes, "session buffer"))) return rc;
        if (b.zero) HIP_OK(hipMemset(b.m->p, 0, b.bytes), "session buffer clear");
    }
    HIP_OK(hipHostMalloc((void**)&s->records, ((size_t)capacity + 2) * sizeof(StepRecord), hipHostMallocMapped),
           "step records");
    std::memset(s->records, 0, ((size_t)capacity + 2) * sizeof(StepRecord));
    HIP_OK(hipHostGetDevicePointer((void**)&s->records_dev, s->records, 0), "step records mapping");
    HIP_OK(hipHostMalloc((void**)&s->state_host, ST_WORDS * 4, hipHostMallocDefault), "state staging");
    s->events.resize(AF_MAX_NEW_TOKENS);
    for (auto& e : s->events) HIP_OK(hipEventCreate(&e), "event");
    HIP_OK(hipEventCreate(&s->ev_start), "event");
    s->attn_xl = attn_xcd_local();
    if ((rc = setup_step(*s))) return rc;
    // A model whose step mixes step-kernel runs with per-operation layers is launched directly:
    // replays of its captured step faulted on the host inside hipGraphLaunch under a rocprofv3
    // kernel trace (cause not established), and without a profiler it decodes at the same rate
    // either way (at most kDecodeAhead steps are queued ahead, so launch costs are hidden).
    if (s->use_step && s->segmented()) s->use_graphs = false;
    HIP_OK(hipDeviceSynchronize(), "session upload");
    if (s->use_graphs) {
        // the step kernel and the head (decode), or the step kernel alone (prefill); on the
        // per-operation path every layer's kernels.  No timeline memset is recorded: the timer
        // that adds it is only set around direct launches (af_session_profile).
        if ((rc = s->capture(true, s->decode_graph, s->decode_exec))) return rc;
        if ((rc = s->capture(false, s->prefill_graph, s->prefill_exec))) return rc;
    }
    HIP_OK(hipStreamSynchronize(s->stream), "session ready");
    *out = s.release();
    return AF_OK;
}

}  // namespace

extern "C" {

int af_session_open(const af_layer_weights* layers, uint32_t n_layers, const af_output_head* head,
                    uint32_t capacity, af_session** out) {
    return open_session(layers, n_layers, head, capacity, out);
}

void af_session_close(af_session* s) { delete s; }

int af_session_speculation(const af_session* s, uint64_t* passes, uint64_t* drafted, uint64_t* accepted) {
    if (!s || !passes || !drafted || !accepted) return fail(AF_ERR_INVALID, "null argument");
    *passes = s->spec_passes;
    *drafted = s->spec_drafted;
    *accepted = s->spec_accepted;
    return AF_OK;
}

int af_session_reset(af_session* s) {
    if (!s) return fail(AF_ERR_INVALID, "null session");
    if (s->poisoned) return fail(AF_ERR_POISONED, "invalid HIP session; restart the chat");
    s->cached.clear();
    s->consumed = 0;
    return AF_OK;
}

}  // extern "C"

namespace {

// Prompt-lookup draft (crates/cuda-backend/src/stack.rs:1491-1511): the tokens that followed the most
// recent earlier occurrence of the history's last 3 tokens, at most `limit` of them.
std::vector<uint32_t> draft_lookup(const std::vector<uint32_t>& h, size_t limit) {
    constexpr size_t gram = 3;
    if (h.size() <= gram || limit == 0) return {};
    const size_t tail = h.size() - gram;
    for (size_t start = tail; start-- > 0;) {
        if (std::equal(h.begin() + start, h.begin() + start + gram, h.begin() + tail)) {
            const size_t from = start + gram, end = std::min(from + limit, h.size());
            if (from < end) return std::vector<uint32_t>(h.begin() + from, h.begin() + end);
        }
    }
    return {};
}

// The decode loop of GenerationSession::generate with speculation (stack.rs:1252-1338), after the
// prefill has left position P - 1 (or, with nothing pending, the last consumed position's head input)
// to run.  Each round emits the pending greedy token; with a draft, the token and its draft go through
// the batched layers at once, the head runs over the positions (up to kHeadBatchMax per launch, the
// table read once per launch) until the first prediction that differs from the draft, the
// matching draft tokens are emitted, and the caches keep only their
// positions (the rest are overwritten later: a local ring holds window + kBatchMax slots).  The
// emitted ids are the greedy ids of plain decoding, up to the arithmetic of the batched layers.
int speculate(af_session* s, const uint32_t* prompt, size_t n_prompt, const uint32_t* stop, size_t n_stop,
              uint32_t max_new, af_token_fn on_token, void* user, uint32_t* ids_out, size_t* n_out,
              int32_t* stopped_out, af_generation_stats* stats, Clock::time_point started, double prefill_ms,
              size_t cached_tokens) {
    hipStream_t st = s->stream;
    const size_t H = s->hidden;
    const uint32_t P = (uint32_t)n_prompt;
    int rc;
    if ((rc = s->ensure_batch())) return rc;
    auto is_stop = [&](uint32_t id) { return std::find(stop, stop + n_stop, id) != stop + n_stop; };
    // One decode step on the token at `pos` (already in IDS): step kernel and head in step mode (no
    // stop ids on the device); returns the head's id for pos + 1.
    uint32_t pos = 0;
    auto step = [&](uint32_t& out) -> int {
        for (int attempt = 0; attempt < 2; ++attempt) {
            int r = s->set_state(pos, 0);
            if (r) return r;
            HIP_OK(s->run_step(true), "decode step");
            HIP_OK(hipStreamSynchronize(st), "decode step");
            const volatile StepRecord* vr = s->records + pos + 1;
            if (vr->done) {
                if (vr->bad) return fail(AF_ERR_NONFINITE, "non-finite logits or invalid greedy id");
                out = vr->id;
                ++pos;
                return AF_OK;
            }
            bool timed_out = false;
            if ((r = s->step_timed_out(timed_out, nullptr))) return r;
            if (!timed_out || attempt) break;
            if ((r = s->fall_back())) return r;
        }
        return fail(AF_ERR_DEVICE, "decode step did not complete");
    };
    // The head on hidden state x (down output) and residual h; non-step mode, result in RESULT.
    auto head = [&](const float* x, const float* h, uint32_t& out) -> int {
        HeadArgs a = s->head_args(false, false);
        a.in.x = x;
        a.in.res = h;
        HIP_OK(launch_head(a, IN_RESID, s->head_blocks, st), "head");
        uint32_t res[2] = {0, 0};
        HIP_OK(hipMemcpyAsync(res, s->RESULT.p, sizeof(res), hipMemcpyDeviceToHost, st), "head result");
        HIP_OK(hipStreamSynchronize(st), "head");
        if (res[1]) return fail(AF_ERR_NONFINITE, "non-finite logits or invalid greedy id");
        out = res[0];
        return AF_OK;
    };
    uint32_t next = 0;
    if (P == s->consumed) {  // nothing pending: the head on the last consumed position's state
        pos = s->consumed;
        if ((rc = head(s->D.as<float>(), s->H.as<float>(), next))) return rc;
    } else {
        pos = P - 1;
        if ((rc = step(next))) return rc;
    }
    std::vector<uint32_t> history(prompt, prompt + n_prompt), ids, batch;
    bool stopped = false;
    double first_ms = 0, last_ms = 0;
    auto emit = [&](uint32_t id) {
        const double t = ms_since(started);
        if (ids.empty()) first_ms = t;
        last_ms = t;
        ids.push_back(id);
        history.push_back(id);
        if (on_token) on_token(user, id);
    };
    // A verification pass costs a few decode steps, so after a pass that accepts nothing the next
    // `skip` tokens are decoded without drafting (doubling on each further miss, reset by a hit);
    // the ids are the same either way, up to the rounding of the batched layers' predictions.
    uint32_t skip = 0, backoff = 0;
    while (ids.size() < max_new) {
        if (is_stop(next)) {
            stopped = true;
            break;
        }
        emit(next);
        const size_t remaining = max_new - ids.size();
        const size_t room = s->capacity > pos + 1 ? s->capacity - (pos + 1) : 0;
        const size_t limit = std::min({remaining, room, (size_t)s->spec_depth, (size_t)kVerifyMax - 1});
        std::vector<uint32_t> draft;
        if (skip) --skip;
        else draft = draft_lookup(history, limit);
        if (draft.empty()) {
            HIP_OK(hipMemcpyAsync(s->IDS.as<uint32_t>() + pos, &next, 4, hipMemcpyHostToDevice, st), "id upload");
            if ((rc = step(next))) return rc;
            if (remaining == 0) break;
            continue;
        }
        const uint32_t base = pos, T = (uint32_t)draft.size() + 1;
        batch.assign(1, next);
        batch.insert(batch.end(), draft.begin(), draft.end());
        HIP_OK(hipMemcpyAsync(s->IDS.as<uint32_t>() + base, batch.data(), (size_t)T * 4, hipMemcpyHostToDevice, st),
               "draft upload");
        HIP_OK(s->enqueue_batch(base, T, nullptr), "verification pass");
        // position i's prediction, until the first that differs from draft[i]: the head over up to
        // kHeadBatchMax positions per launch (the table read once per launch), launches stopping
        // at the first batch that holds a difference
        size_t keep = 0;
        uint32_t predicted = 0;
        bool differs = false;
        for (uint32_t i0 = 0; i0 < T && !differs; i0 += kHeadBatchMax) {
            const uint32_t nv = std::min<uint32_t>(kHeadBatchMax, T - i0);
            HeadArgs ha = s->head_args(false, false);
            ha.in.x = s->DB.as<float>() + i0 * H;
            ha.in.res = s->HB.as<float>() + i0 * H;
            HIP_OK(launch_head_batch(ha, nv, (uint32_t)H, s->head_blocks, st), "verification head");
            uint32_t res[2 * kHeadBatchMax] = {};
            HIP_OK(hipMemcpyAsync(res, s->RESULT.p, (size_t)nv * 8, hipMemcpyDeviceToHost, st), "head results");
            HIP_OK(hipStreamSynchronize(st), "verification head");
            for (uint32_t j = 0; j < nv; ++j) {
                if (res[2 * j + 1]) return fail(AF_ERR_NONFINITE, "non-finite logits or invalid greedy id");
                predicted = res[2 * j];
                const uint32_t i = i0 + j;
                if (i == draft.size() || predicted != draft[i]) {
                    differs = true;
                    break;
                }
                ++keep;
            }
        }
        size_t emitted = 0;
        for (; emitted < keep; ++emitted) {
            if (is_stop(draft[emitted])) {
                stopped = true;
                break;
            }
            emit(draft[emitted]);
        }
        // the state after position base + emitted, where the next step or head continues
        pos = base + 1 + (uint32_t)emitted;
        HIP_OK(hipMemcpyAsync(s->D.p, s->DB.as<float>() + emitted * H, H * 4, hipMemcpyDeviceToDevice, st), "state");
        HIP_OK(hipMemcpyAsync(s->H.p, s->HB.as<float>() + emitted * H, H * 4, hipMemcpyDeviceToDevice, st), "state");
        HIP_OK(hipStreamSynchronize(st), "verification pass");
        s->spec_drafted += draft.size();
        s->spec_accepted += keep;
        ++s->spec_passes;
        if (keep == 0) {
            backoff = std::min<uint32_t>(2 * backoff + 2, 32);
            skip = backoff;
        } else {
            backoff = 0;
        }
        if (stopped) break;
        next = predicted;
    }
    for (size_t i = 0; i < ids.size(); ++i) ids_out[i] = ids[i];
    s->cached.assign(prompt, prompt + n_prompt);
    s->cached.insert(s->cached.end(), ids.begin(), ids.end());
    s->consumed = pos;
    s->poisoned = false;
    if (n_out) *n_out = ids.size();
    if (stopped_out) *stopped_out = stopped;
    if (stats) {
        stats->prompt_tokens = n_prompt - cached_tokens;
        stats->cached_tokens = cached_tokens;
        stats->prefill_ms = prefill_ms;
        stats->has_first_token = !ids.empty();
        stats->first_token_ms = ids.empty() ? 0.0 : first_ms;
        stats->decode_tokens = ids.empty() ? 0 : ids.size() - 1;
        stats->decode_ms = ids.empty() ? 0.0 : last_ms - first_ms;
        stats->total_ms = ms_since(started);
    }
    return AF_OK;
}

// GenerationSession::generate (crates/cuda-backend/src/stack.rs:1171-1386).  With a timer the
// decode steps are launched directly with an event pair around every kernel (no stop ids).
// Decode steps queued on the stream ahead of the one whose id is being read back.
constexpr uint32_t kDecodeAhead = 8;

int generate_core(af_session* s, const uint32_t* prompt, size_t n_prompt, const uint32_t* stop, size_t n_stop,
                  uint32_t max_new, af_token_fn on_token, void* user, uint32_t* ids_out, size_t* n_out,
                  int32_t* stopped_out, af_generation_stats* stats, KernelTimer* timer) {
    if (!s) return fail(AF_ERR_INVALID, "null session");
    if (n_out) *n_out = 0;
    if (stopped_out) *stopped_out = 0;
    if (s->poisoned) return fail(AF_ERR_POISONED, "invalid HIP session; restart the chat");
    // stack.rs:1184-1194
    bool ok = prompt && n_prompt > 0 && max_new >= 1 && max_new <= AF_MAX_NEW_TOKENS &&
              n_prompt + max_new <= s->capacity && (timer || (stop && n_stop > 0)) && n_stop <= kMaxStopIds &&
              ids_out && n_prompt >= s->cached.size();
    for (size_t i = 0; ok && i < n_prompt; ++i) ok = prompt[i] < s->vocabulary;
    for (size_t i = 0; ok && i < n_stop; ++i) ok = stop[i] < s->vocabulary;
    for (size_t i = 0; ok && i < s->cached.size(); ++i) ok = prompt[i] == s->cached[i];
    if (!ok) return fail(AF_ERR_INVALID, "prompt, KV prefix or session capacity incompatible");

    const auto started = Clock::now();
    const size_t cached_tokens = s->cached.size();
    s->poisoned = true;
    const uint32_t P = (uint32_t)n_prompt, pend = P - s->consumed;
    hipStream_t st = s->stream;
    HIP_OK(hipMemcpyAsync(s->IDS.as<uint32_t>() + s->consumed, prompt + s->consumed, (size_t)pend * 4,
                          hipMemcpyHostToDevice, st),
           "prompt upload");
    if (n_stop) HIP_OK(hipMemcpyAsync(s->STOPS.p, stop, n_stop * 4, hipMemcpyHostToDevice, st), "stop ids upload");
    std::memset(s->records + P, 0, (size_t)(s->capacity + 2 - P) * sizeof(StepRecord));
    // Positions consumed .. P - 2 fill the KV caches: in batches through the batched layers, or one
    // step-kernel launch (graph replay) each; the decode steps then start at position P - 1.
    const bool batched = s->prefill_batch > 1 && pend > 1 && !timer;
    int rc = s->set_state(batched ? P - 1 : pend == 0 ? s->consumed - 1 : s->consumed, (uint32_t)n_stop);
    if (rc) return rc;
    if (batched) {
        if ((rc = s->ensure_batch())) return rc;
        HIP_OK(s->prefill_batched(s->consumed, P - 1, s->prefill_batch), "batched prefill");
    } else {
        for (uint32_t i = 0; i + 1 < pend; ++i) HIP_OK(s->run_step(false), "prefill step");
    }
    HIP_OK(hipStreamSynchronize(st), "prefill");
    if (pend > 1 && !batched) {  // a timed-out step kernel: rerun from its position on the per-operation kernels
        bool timed_out = false;
        uint32_t at = 0;
        if ((rc = s->step_timed_out(timed_out, &at))) return rc;
        if (timed_out) {
            if ((rc = s->fall_back()) || (rc = s->set_state(at, (uint32_t)n_stop))) return rc;
            for (uint32_t q = at; q + 1 < P; ++q) HIP_OK(s->run_step(false), "prefill step");
            HIP_OK(hipStreamSynchronize(st), "prefill");
        }
    }
    const double prefill_ms = ms_since(started);
    if (s->speculative && !timer)
        return speculate(s, prompt, n_prompt, stop, n_stop, max_new, on_token, user, ids_out, n_out, stopped_out, stats,
                         started, prefill_ms, cached_tokens);
    const double start_offset = ms_since(started);
    HIP_OK(hipEventRecord(s->ev_start, st), "event");
    // Enqueue the decode steps from k0 on; each step's head writes its id and flags to mapped host
    // memory, and a stop id makes the remaining steps return at once.
    // Steps k0 .. k1 - 1 onto the stream.  At most kDecodeAhead steps are queued ahead of the one
    // being read back: the GPU never waits for the host (a step takes milliseconds, a launch
    // microseconds), and a call of many steps does not put thousands of kernel dispatches in flight
    // at once (a 128-step call of a model whose decode graph holds 49 kernels would queue 6,272).
    uint32_t queued = 0;
    auto enqueue_range = [&](uint32_t k0, uint32_t k1) -> int {
        s->timer = timer;
        for (uint32_t k = k0; k < k1; ++k) {
            s->host_pos = P - 1 + k;
            hipError_t e;
            if (k == 0 && pend == 0)
                e = s->timed(K_HEAD, (double)s->head.rows * (s->head.columns / 256) * 210.0 + 12.0 * s->hidden, [&] {
                    return launch_head(s->head_args(true, false), IN_RESID, s->head_blocks, st);
                });
            else
                e = timer ? s->enqueue_step(true) : s->run_step(true);
            if (e == hipSuccess) e = hipEventRecord(s->events[k], st);
            if (e != hipSuccess) {
                s->timer = nullptr;
                return fail(AF_ERR_DEVICE, std::string("decode step: ") + hipGetErrorString(e));
            }
        }
        s->timer = nullptr;
        queued = std::max(queued, k1);
        return AF_OK;
    };
    if ((rc = enqueue_range(0, std::min(max_new, kDecodeAhead)))) return rc;
    std::vector<uint32_t> ids;
    bool stopped = false, bad = false;
    double first_ms = 0, last_ms = 0;
    for (uint32_t k = 0; k < max_new; ++k) {
        HIP_OK(hipEventSynchronize(s->events[k]), "decode step");
        if (queued < max_new && (rc = enqueue_range(queued, queued + 1))) return rc;
        const volatile StepRecord* vr = s->records + P + k;
        StepRecord r;
        r.id = vr->id;
        r.bad = vr->bad;
        r.stop = vr->stop;
        r.done = vr->done;
        if (!r.done && s->use_step) {
            // step k's kernel may have timed out (its head then returned at once): rerun steps k..
            // on the per-operation kernels from the step's position
            HIP_OK(hipStreamSynchronize(st), "decode step");
            bool timed_out = false;
            if ((rc = s->step_timed_out(timed_out, nullptr))) return rc;
            if (timed_out) {
                queued = k;
                if ((rc = s->fall_back()) || (rc = s->set_state(P - 1 + k, (uint32_t)n_stop)) ||
                    (rc = enqueue_range(k, std::min(max_new, k + kDecodeAhead))))
                    return rc;
                --k;
                continue;
            }
        }
        float t = 0;
        (void)hipEventElapsedTime(&t, s->ev_start, s->events[k]);
        if (!r.done || r.bad) {
            bad = true;
            break;
        }
        if (r.stop) {
            stopped = true;
            break;
        }
        if (k == 0) first_ms = start_offset + t;
        last_ms = start_offset + t;
        ids.push_back(r.id);
        if (on_token) on_token(user, r.id);
    }
    HIP_OK(hipStreamSynchronize(st), "generation");
    if (bad) {
        uint32_t words[ST_WORDS] = {};
        HIP_OK(hipMemcpy(words, s->STATE.p, sizeof(words), hipMemcpyDeviceToHost), "state download");
        if (words[ST_BAD] == 2u) return fail(AF_ERR_DEVICE, "decode step grid barrier did not complete");
        return fail(AF_ERR_NONFINITE, "non-finite logits or invalid greedy id");
    }
    for (size_t i = 0; i < ids.size(); ++i) ids_out[i] = ids[i];
    s->cached.assign(prompt, prompt + n_prompt);
    s->cached.insert(s->cached.end(), ids.begin(), ids.end());
    // The last generated token is consumed by the next call's first step.
    s->consumed = stopped ? (uint32_t)s->cached.size() : (uint32_t)s->cached.size() - 1;
    s->poisoned = false;
    if (n_out) *n_out = ids.size();
    if (stopped_out) *stopped_out = stopped;
    if (stats) {
        stats->prompt_tokens = n_prompt - cached_tokens;
        stats->cached_tokens = cached_tokens;
        stats->prefill_ms = prefill_ms;
        stats->has_first_token = !ids.empty();
        stats->first_token_ms = ids.empty() ? 0.0 : first_ms;
        stats->decode_tokens = ids.empty() ? 0 : ids.size() - 1;
        stats->decode_ms = ids.empty() ? 0.0 : last_ms - first_ms;
        stats->total_ms = ms_since(started);
    }
    return AF_OK;
}

}  // namespace

extern "C" {

int af_session_generate(af_session* s, const uint32_t* prompt, size_t n_prompt, const uint32_t* stop,
                        size_t n_stop, uint32_t max_new, af_token_fn on_token, void* user, uint32_t* ids_out,
                        size_t* n_out, int32_t* stopped_out, af_generation_stats* stats) {
    return generate_core(s, prompt, n_prompt, stop, n_stop, max_new, on_token, user, ids_out, n_out, stopped_out,
                         stats, nullptr);
}

int af_session_profile(af_session* s, const uint32_t* prompt, size_t n_prompt, uint32_t max_new, uint32_t* ids_out,
                       size_t* n_out, af_kernel_timing* timings, size_t capacity, size_t* n_timings) {
    if (!timings || !n_timings || capacity < K_KINDS) return fail(AF_ERR_INVALID, "timing output too small");
    KernelTimer timer;
    if (s && s->use_step && !s->poisoned && !s->segmented()) {
        const size_t bytes = (size_t)max_new * s->clock_words() * 8;
        if (s->CLOCK.bytes < bytes) {
            int r = dev_alloc(s->CLOCK, bytes, "step timeline");
            if (r) return r;
        }
        // the first half of the steps run plain ("layers"), the rest write the timeline
        // ("layers_timeline" and the phase entries)
        s->clock_steps = max_new - max_new / 2;
        s->clock_skip = max_new / 2;
        s->clock_used = 0;
    }
    int rc = generate_core(s, prompt, n_prompt, nullptr, 0, max_new, nullptr, nullptr, ids_out, n_out, nullptr,
                           nullptr, &timer);
    const uint32_t timed_steps = s ? s->clock_used : 0;
    if (s) s->clock_steps = s->clock_skip = 0;
    if (rc) return rc;
    for (int k = 0; k < K_KINDS; ++k) {
        std::memset(&timings[k], 0, sizeof(timings[k]));
        std::snprintf(timings[k].name, sizeof(timings[k].name), "%s", kKindNames[k]);
    }
    for (size_t i = 0; i < timer.used; ++i) {
        const auto& r = timer.recs[i];
        float ms = 0;
        HIP_OK(hipEventElapsedTime(&ms, r.a, r.b), "kernel timing");
        af_kernel_timing& t = timings[r.kind];
        t.launches += 1;
        t.total_ms += ms;
        t.bytes_per_launch += r.bytes;
    }
    // Step kernel timelines: a phase runs from its opening barrier's departure (workgroup 0) to
    // the last workgroup's arrival at the closing barrier; the barrier itself from that arrival
    // to workgroup 0's departure.  "<phase>.<mark>" entries split the slowest workgroup's phase
    // at its marks (time since its previous mark), and "<phase>.mean" is the mean over
    // workgroups of their own start-to-arrival time.
    std::vector<af_kernel_timing> extra;
    if (timed_steps) {
        const size_t words = s->clock_words();
        std::vector<uint64_t> clk((size_t)timed_steps * words);
        HIP_OK(hipMemcpy(clk.data(), s->CLOCK.p, clk.size() * 8, hipMemcpyDeviceToHost), "timeline download");
        const uint32_t G = s->step_grid, nb = s->barriers();
        const double tick_ms = 1e-5;  // 100 MHz
        static const char* const kMarkNames[kStepMarks] = {"start", "stage", "digits", "stream", "store", "tail", "pre", "consume"};
        static const int kOrder[] = {M_START, M_STAGED, M_DIGITS, M_CONSUMED, M_STREAMED, M_STORED, M_PRE, M_ARRIVE};
        auto entry = [&](const std::string& name) -> af_kernel_timing& {
            for (auto& t : extra)
                if (name == t.name) return t;
            af_kernel_timing t{};
            std::snprintf(t.name, sizeof(t.name), "%s", name.c_str());
            extra.push_back(t);
            return extra.back();
        };
        for (uint32_t st = 0; st < timed_steps; ++st) {
            const uint64_t* c = clk.data() + (size_t)st * words;
            auto ev = [&](uint32_t ph, int mark, uint32_t b) { return c[((size_t)ph * kStepMarks + mark) * G + b]; };
            for (uint32_t p = 0; p <= nb; ++p) {
                uint32_t crit = 0;
                uint64_t arrive = 0;
                double mean = 0;
                for (uint32_t b = 0; b < G; ++b) {
                    const uint64_t t = ev(p, M_ARRIVE, b);
                    if (t > arrive) {
                        arrive = t;
                        crit = b;
                    }
                    const uint64_t t0 = ev(p, M_START, b);
                    mean += t > t0 ? (double)(t - t0) : 0.0;
                }
                const uint64_t open = ev(p, M_START, 0);
                const int kind = K_QKV + (int)(p % 5);
                timings[kind].launches += 1;
                timings[kind].total_ms += (double)(arrive - std::min(arrive, open)) * tick_ms;
                const std::string base = kKindNames[kind];
                af_kernel_timing& m = entry(base + ".mean");
                m.launches += 1;
                m.total_ms += mean / G * tick_ms;
                uint64_t prev = ev(p, M_START, crit);
                for (int mk : kOrder) {
                    if (mk == M_START) continue;
                    const uint64_t t = ev(p, mk, crit);
                    if (!t || t < prev) continue;
                    af_kernel_timing& e = entry(base + "." + kMarkNames[mk == M_ARRIVE ? 5 : mk]);
                    e.launches += 1;
                    e.total_ms += (double)(t - prev) * tick_ms;
                    prev = t;
                }
                // each mark's mean offset from the workgroup's own phase start ("<phase>.<mark>@")
                for (int mk = M_STAGED; mk < kStepMarks; ++mk) {
                    if (mk == M_ARRIVE) continue;
                    double sum = 0;
                    uint32_t cnt = 0;
                    for (uint32_t b = 0; b < G; ++b) {
                        const uint64_t t0 = ev(p, M_START, b), t = ev(p, mk, b);
                        if (t && t >= t0) {
                            sum += (double)(t - t0);
                            ++cnt;
                        }
                    }
                    if (cnt) {
                        af_kernel_timing& e = entry(base + "." + kMarkNames[mk] + "@");
                        e.launches += 1;
                        e.total_ms += sum / cnt * tick_ms;
                    }
                }
                // the same split averaged over every workgroup ("<phase>.<mark>~")
                for (uint32_t b = 0; b < G; ++b) {
                    uint64_t pv = ev(p, M_START, b);
                    for (int mk : kOrder) {
                        if (mk == M_START) continue;
                        const uint64_t t = ev(p, mk, b);
                        if (!t || t < pv) continue;
                        af_kernel_timing& e = entry(base + "." + kMarkNames[mk == M_ARRIVE ? 5 : mk] + "~");
                        e.launches += 1;
                        e.total_ms += (double)(t - pv) * tick_ms;
                        pv = t;
                    }
                }
                if (p < nb) {
                    const uint64_t depart = ev(p + 1, M_START, 0);
                    timings[K_BARRIER].launches += 1;
                    timings[K_BARRIER].total_ms += (double)(depart - std::min(depart, arrive)) * tick_ms;
                }
            }
        }
        const LayerDev& L0 = s->layers[0];
        timings[K_QKV].bytes_per_launch += af_session::q4_bytes(L0.qkv) * timings[K_QKV].launches;
        timings[K_OPROJ].bytes_per_launch += af_session::q4_bytes(L0.o) * timings[K_OPROJ].launches;
        timings[K_GATEUP].bytes_per_launch +=
            (af_session::q4_bytes(L0.gate) + af_session::q4_bytes(L0.up)) * timings[K_GATEUP].launches;
        timings[K_DOWN].bytes_per_launch += af_session::q4_bytes(L0.down) * timings[K_DOWN].launches;
    }
    for (int k = 0; k < K_KINDS; ++k)
        if (timings[k].launches) timings[k].bytes_per_launch /= (double)timings[k].launches;
    size_t n = K_KINDS;
    for (const auto& e : extra)
        if (n < capacity) timings[n++] = e;
    *n_timings = n;
    return AF_OK;
}

int af_generate(const af_layer_weights* layers, uint32_t n_layers, const af_output_head* head,
                const uint32_t* prompt, size_t n_prompt, const uint32_t* stop, size_t n_stop, uint32_t max_new,
                uint32_t* ids_out, size_t* n_out, int32_t* stopped, af_generation_stats* stats) {
    // stack.rs:820-833
    if (n_prompt > 256 || max_new < 1 || max_new > AF_MAX_NEW_TOKENS)
        return fail(AF_ERR_INVALID, "invalid generation configuration");
    af_session* s = nullptr;
    int rc = open_session(layers, n_layers, head, (uint32_t)n_prompt + max_new, &s);
    if (rc) return rc;
    rc = af_session_generate(s, prompt, n_prompt, stop, n_stop, max_new, nullptr, nullptr, ids_out, n_out, stopped,
                             stats);
    delete s;
    return rc;
}

int af_session_trace(af_session* s, const uint32_t* ids, size_t n, float* layer_outputs, uint16_t* kv_appended,
                     float* logits, float* hidden) {
    if (!s) return fail(AF_ERR_INVALID, "null session");
    if (s->poisoned) return fail(AF_ERR_POISONED, "invalid HIP session; restart the chat");
    if (!ids || n == 0 || s->cached.size() + n > s->capacity)
        return fail(AF_ERR_INVALID, "trace ids exceed the session capacity");
    for (size_t i = 0; i < n; ++i)
        if (ids[i] >= s->vocabulary) return fail(AF_ERR_INVALID, "token id outside the vocabulary");
    s->poisoned = true;
    hipStream_t st = s->stream;
    const size_t nl = s->layers.size(), H = s->hidden;
    int rc;
    if (layer_outputs && (rc = grow(s->SNAP, nl * H * 4, false, "trace buffer"))) return rc;
    const size_t kvr = s->max_kv_rows, kv_bytes = nl * 2 * kvr * 2;
    if (kv_appended && (rc = grow(s->KVSNAP, kv_bytes, true, "trace buffer"))) return rc;
    // Tokens generated but not yet run through the layers go first, unreported.
    const size_t pend = s->cached.size() - s->consumed;
    std::vector<uint32_t> run(s->cached.begin() + s->consumed, s->cached.end());
    run.insert(run.end(), ids, ids + n);
    HIP_OK(hipMemcpyAsync(s->IDS.as<uint32_t>() + s->consumed, run.data(), run.size() * 4, hipMemcpyHostToDevice, st),
           "ids upload");
    if (s->trace_batch > 1) {
        // every position through the batched layers: layer outputs and appended K/V per batch
        if ((rc = s->ensure_batch())) return rc;
        if (layer_outputs && (rc = grow(s->SNAP, (size_t)kBatchMax * nl * H * 4, false, "trace buffer"))) return rc;
        const uint32_t B = s->trace_batch, first = s->consumed + (uint32_t)pend;
        HIP_OK(s->prefill_batched(s->consumed, first, B), "trace batch");
        uint32_t T = 0;
        for (size_t p = 0; p < n; p += T) {
            T = (uint32_t)std::min<size_t>(B, n - p);
            HIP_OK(s->enqueue_batch(first + (uint32_t)p, T, layer_outputs ? s->SNAP.as<float>() : nullptr),
                   "trace batch");
            if (layer_outputs)
                HIP_OK(hipMemcpyAsync(layer_outputs + p * nl * H, s->SNAP.p, (size_t)T * nl * H * 4,
                                      hipMemcpyDeviceToHost, st),
                       "trace download");
            for (uint32_t t = 0; kv_appended && t < T; ++t) {
                for (uint32_t l = 0; l < nl; ++l) {
                    const LayerDev& L = s->layers[l];
                    const size_t slot = (first + p + t) % L.ring, row = (size_t)L.width * 2;
                    uint8_t* dst = s->KVSNAP.as<uint8_t>() + (size_t)l * 2 * kvr * 2;
                    HIP_OK(hipMemcpy2DAsync(dst, row, L.kcache.as<uint8_t>() + slot * row, (size_t)L.ring * row, row,
                                            L.kv_heads, hipMemcpyDeviceToDevice, st),
                           "trace K/V copy");
                    HIP_OK(hipMemcpy2DAsync(dst + kvr * 2, row, L.vcache.as<uint8_t>() + slot * row,
                                            (size_t)L.ring * row, row, L.kv_heads, hipMemcpyDeviceToDevice, st),
                           "trace K/V copy");
                }
                HIP_OK(hipMemcpyAsync(kv_appended + (p + t) * nl * 2 * kvr, s->KVSNAP.p, kv_bytes,
                                      hipMemcpyDeviceToHost, st),
                       "trace download");
            }
        }
        // head on the last position's final hidden state (raw logits)
        HeadArgs h = s->head_args(false, true);
        h.in.x = s->DB.as<float>() + (size_t)(T - 1) * H;
        h.in.res = s->HB.as<float>() + (size_t)(T - 1) * H;
        HIP_OK(launch_head(h, IN_RESID, s->head_blocks, st), "trace head");
        if (logits)
            HIP_OK(hipMemcpyAsync(logits, s->LOGITS.p, (size_t)s->vocabulary * 4, hipMemcpyDeviceToHost, st), "logits");
        if (hidden) HIP_OK(hipMemcpyAsync(hidden, s->X.p, H * 4, hipMemcpyDeviceToHost, st), "hidden");
        HIP_OK(hipStreamSynchronize(st), "trace");
    } else
    // A step kernel that times out makes the session fall back to the per-operation kernels, and
    // the whole trace runs again there (it rewrites the same K/V slots).
    for (int attempt = 0; attempt < 2; ++attempt) {
    if ((rc = s->set_state(s->consumed, 0))) return rc;
    // step: one step-kernel launch per position; otherwise the layers one by one (per-operation
    // kernels, and the step kernel's runs of a segmented session)
    const bool step = s->use_step && !s->segmented();
    for (size_t i = 0; i < pend; ++i) {
        if (step) {
            HIP_OK(launch_step(s->step_args(0, true, nullptr), s->group, s->step_grid, s->step_lds, st), "trace step");
        } else {
            HIP_OK(s->enqueue_layers(), "trace layers");
            HIP_OK(launch_advance(s->STATE.as<uint32_t>(), st), "trace advance");
        }
    }
    // layer l's output: (rms(D) post_ffn + H) * scale after layer l
    auto snapshot = [&](uint32_t l) -> hipError_t {
        InputStage r{};
        r.x = s->D.as<float>();
        r.res = s->H.as<float>();
        r.w_a = s->layers[l].post_ffn.as<float>();
        r.eps_a = s->layers[l].post_ffn_eps;
        r.scale = s->layers[l].layer_scale;
        return launch_resid(r, s->hidden, s->SNAP.as<float>() + l * H, st);
    };
    auto kv_copy = [&](uint32_t l, size_t t) -> hipError_t {
        const LayerDev& L = s->layers[l];
        const size_t slot = (s->consumed + pend + t) % L.ring, row = (size_t)L.width * 2;
        uint8_t* dst = s->KVSNAP.as<uint8_t>() + (size_t)l * 2 * kvr * 2;
        hipError_t e = hipMemcpy2DAsync(dst, row, L.kcache.as<uint8_t>() + slot * row, (size_t)L.ring * row, row,
                                        L.kv_heads, hipMemcpyDeviceToDevice, st);
        if (e != hipSuccess) return e;
        return hipMemcpy2DAsync(dst + kvr * 2, row, L.vcache.as<uint8_t>() + slot * row, (size_t)L.ring * row, row,
                                L.kv_heads, hipMemcpyDeviceToDevice, st);
    };
    for (size_t t = 0; t < n; ++t) {
        if (step) {
            // the step kernel writes layers 0..L-2's outputs; the last comes from D and H after it
            HIP_OK(launch_step(s->step_args(0, true, layer_outputs ? s->SNAP.as<float>() : nullptr), s->group,
                               s->step_grid, s->step_lds, st),
                   "trace step");
            if (layer_outputs) HIP_OK(snapshot(nl - 1), "trace snapshot");
            if (kv_appended)
                for (uint32_t l = 0; l < nl; ++l) HIP_OK(kv_copy(l, t), "trace K/V copy");
        } else {
            for (uint32_t l = 0; l < nl;) {
                if (s->use_step && s->in_step[l]) {
                    // a run writes its layers' outputs but the last, which comes from D and H after it
                    const uint32_t k = (uint32_t)s->run_at[l], n_run = s->runs[k].n;
                    HIP_OK(launch_step(s->step_args(k, false, layer_outputs ? s->SNAP.as<float>() + l * H : nullptr),
                                       s->group, s->step_grid, s->step_lds, st),
                           "trace step");
                    if (kv_appended)
                        for (uint32_t j = l; j < l + n_run; ++j) HIP_OK(kv_copy(j, t), "trace K/V copy");
                    if (layer_outputs) HIP_OK(snapshot(l + n_run - 1), "trace snapshot");
                    l += n_run;
                } else {
                    HIP_OK(s->enqueue_layer(l, true), "trace layer");
                    if (kv_appended) HIP_OK(kv_copy(l, t), "trace K/V copy");
                    if (layer_outputs) HIP_OK(snapshot(l), "trace snapshot");
                    ++l;
                }
            }
        }
        if (layer_outputs)
            HIP_OK(hipMemcpyAsync(layer_outputs + t * nl * H, s->SNAP.p, nl * H * 4, hipMemcpyDeviceToHost, st),
                   "trace download");
        if (kv_appended)
            HIP_OK(hipMemcpyAsync(kv_appended + t * nl * 2 * kvr, s->KVSNAP.p, kv_bytes, hipMemcpyDeviceToHost, st),
                   "trace download");
        if (!step && t + 1 < n) HIP_OK(launch_advance(s->STATE.as<uint32_t>(), st), "trace advance");
    }
    // head on the last token: raw logits, no state change (the step kernel already advanced)
    HeadArgs h = s->head_args(false, true);
    HIP_OK(launch_head(h, IN_RESID, s->head_blocks, st), "trace head");
    if (!step) HIP_OK(launch_advance(s->STATE.as<uint32_t>(), st), "trace advance");
    if (logits) HIP_OK(hipMemcpyAsync(logits, s->LOGITS.p, (size_t)s->vocabulary * 4, hipMemcpyDeviceToHost, st), "logits");
    if (hidden) HIP_OK(hipMemcpyAsync(hidden, s->X.p, H * 4, hipMemcpyDeviceToHost, st), "hidden");
    HIP_OK(hipStreamSynchronize(st), "trace");
    bool timed_out = false;
    if ((rc = s->step_timed_out(timed_out, nullptr))) return rc;
    if (!timed_out) break;
    if ((rc = s->fall_back())) return rc;
    }
    s->cached.insert(s->cached.end(), ids, ids + n);
    s->consumed = (uint32_t)s->cached.size();
    s->poisoned = false;
    return AF_OK;
}

}  // extern "C"
