// Persistent decode step for gfx950 (MI355X): all layers of one decode step in one cooperative
// launch of one 512-thread workgroup per CU.  Per layer it runs five phases separated by grid
// barriers: qkv GEMV (residual + RMSNorm prologue), GQA attention over the fp16 KV cache
// (split-K, merged by the last chunk of each KV head), o-proj GEMV, fused gate/up GEMV with
// tanh-GELU, down GEMV.
//
// Why one launch: a layer's five dependent kernels each pay a dispatch, a ramp and a drain,
// and their weight streams cannot start before the previous kernel ends.  Here the weights of
// the next phase, which do not depend on any activation, are requested before each grid
// barrier, so HBM keeps streaming while the barrier and the next phase's input prologue
// resolve.
//
// Wave roles: vector memory loads of one wave return in issue order, so a wave whose weight
// prefetch is in flight cannot see an activation load before the prefetch lands.  Wave 0 of
// every workgroup therefore never prefetches weights: it runs the grid barrier and stages the
// phase's input vectors into LDS (global->LDS DMA), while waves 1-7 stream the weights.  The
// input prologue (norms, exact int8 digit planes) then runs on all 512 threads from LDS.
//
// Coherence: the eight XCDs have private L2 caches.  Activations exchanged between workgroups
// inside the launch are written and read with agent-scope coherent accesses (sc1), the grid
// barrier uses agent-scope atomics, and a store is waited for (s_waitcnt vmcnt(0)) before the
// barrier arrival that publishes it.  Weights, norm vectors and the KV cache rows read here
// were written before the launch began.
#include "device.h"

namespace af {

namespace {

constexpr uint32_t kThreads = 512;
constexpr uint32_t kStreamWaves = 7;  // waves 1..7 stream weights
constexpr int kAhead = 8;             // Q4 super-tiles in flight per streaming wave
constexpr int kSC1 = 16;              // cache policy: agent-scope coherent access
constexpr int kVmWait = 0x0F70;       // s_waitcnt vmcnt(0) with expcnt / lgkmcnt unconstrained
constexpr uint32_t kSpinLimit = 1u << 21;
constexpr uint32_t kMaxUnits = kStepMaxUnits;
constexpr uint32_t kMaxT = 4;         // tile streams per unit (gate/up: 2 tiles of 2 matrices)

// Barrier words, 128 bytes apart: [0] groups done, [32 (g + 1)] arrivals of group g (g < 8,
// workgroups b with b % 8 == g, which share an XCD), [32 * 9] exits.
constexpr uint32_t kBarAll = 0, kBarExit = 32 * 9;

typedef __attribute__((address_space(3))) void* lds_ptr;

__device__ __forceinline__ __amdgpu_buffer_rsrc_t rsrc(const void* p) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(p), 0, 0x7FFFFFFF, 0x00020000);
}
__device__ __forceinline__ uint32_t ldc(const void* base, uint32_t off) {
    return __builtin_amdgcn_raw_buffer_load_b32(rsrc(base), off, 0, kSC1);
}
__device__ __forceinline__ void stc(void* base, uint32_t off, uint32_t v) {
    __builtin_amdgcn_raw_buffer_store_b32(v, rsrc(base), off, 0, kSC1);
}
__device__ __forceinline__ void stc8(void* base, uint32_t off, v2u v) {
    __builtin_amdgcn_raw_buffer_store_b64(v, rsrc(base), off, 0, kSC1);
}
__device__ __forceinline__ void stc16(void* base, uint32_t off, v4u v) {
    __builtin_amdgcn_raw_buffer_store_b128(v, rsrc(base), off, 0, kSC1);
}
__device__ __forceinline__ void wait_vm() { __builtin_amdgcn_s_waitcnt(kVmWait); }

// Wave-level global -> LDS copy of `bytes` (a multiple of 16) with coherent loads; the caller
// waits with wait_vm().
__device__ __forceinline__ void dma(const void* src, uint32_t bytes, uint8_t* lds, uint32_t lane) {
    for (uint32_t off = 0; off < bytes; off += 1024) {
        if (off + lane * 16 < bytes)
            __builtin_amdgcn_global_load_lds(static_cast<const uint8_t*>(src) + off + lane * 16,
                                             (lds_ptr)(lds + off), 16, 0, kSC1);
    }
}

// ---- grid barrier -------------------------------------------------------------------------------

struct Grid {
    uint32_t* bar;
    uint32_t k;       // barriers passed in this launch
    int* ok;          // LDS flag
    uint64_t* clock;  // optional timeline (StepArgs::clock)
};

__device__ __forceinline__ void stamp(const Grid& g, uint32_t e) {
    if (g.clock) g.clock[(size_t)e * gridDim.x + blockIdx.x] = wall_clock64();
}

// All threads call it.  Returns false (in every thread) if the barrier did not complete within
// the spin limit, which only a launch without co-resident workgroups could cause.
__device__ __forceinline__ bool grid_sync(Grid& g) {
    __syncthreads();
    if (threadIdx.x == 0) {
        stamp(g, 1 + 2 * g.k);
        const uint32_t per = gridDim.x / 8, grp = blockIdx.x & 7, k = g.k + 1;
        const uint32_t old =
            __hip_atomic_fetch_add(g.bar + 32 * (1 + grp), 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        if (old + 1 == k * per) __hip_atomic_fetch_add(g.bar + kBarAll, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        uint32_t spins = 0;
        int ok = 1;
        while (__hip_atomic_load(g.bar + kBarAll, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) < 8 * k) {
            __builtin_amdgcn_s_sleep(1);
            if (++spins > kSpinLimit) {
                ok = 0;
                break;
            }
        }
        *g.ok = ok;
        stamp(g, 2 + 2 * g.k);
    }
    __syncthreads();
    ++g.k;
    return *g.ok != 0;
}

// Last workgroup out resets the barrier words for the next launch; with `advance` it also moves
// the session position (a step without the head).
__device__ __forceinline__ void grid_exit(Grid& g, uint32_t* state, bool advance, bool failed) {
    __syncthreads();
    if (threadIdx.x == 0) {
        stamp(g, 1 + 2 * g.k);
        if (failed) {
            __hip_atomic_store(state + ST_BAD, 2u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            __hip_atomic_store(state + ST_STOP, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
        const uint32_t old = __hip_atomic_fetch_add(g.bar + kBarExit, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        if (old == gridDim.x - 1) {
            for (uint32_t i = 0; i < 10; ++i)
                __hip_atomic_store(g.bar + 32 * i, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            if (advance) state[ST_POS] += 1u;
        }
    }
}

// ---- GEMV phases --------------------------------------------------------------------------------

// Rows are grouped into units: one 16-row tile (T = 1), or two tiles of two matrices (T = 4:
// gate tiles 2u, 2u + 1 then up tiles 2u, 2u + 1).  Workgroup b takes units b, b + G, ...
// (at most kMaxUnits); its super-tile work, flattened as (unit, tile stream, super-tile), is
// split evenly over the streaming waves.
struct Job {
    const uint4* codes[2];
    const uint2* scales[2];
    uint32_t nst, units, T;
};

struct Cur {
    uint32_t f, st, ts, k;
};

__device__ __forceinline__ Cur cur_at(uint32_t f, uint32_t nst, uint32_t T) {
    const uint32_t seg = f / nst;
    return Cur{f, f - seg * nst, seg % T, seg / T};
}

__device__ __forceinline__ void cur_next(Cur& c, uint32_t nst, uint32_t T) {
    ++c.f;
    if (++c.st == nst) {
        c.st = 0;
        if (++c.ts == T) {
            c.ts = 0;
            ++c.k;
        }
    }
}

struct Stream {
    Cur ld, cs;
    uint32_t fe;
};

__device__ __forceinline__ uint32_t my_units(uint32_t units) {
    return units > blockIdx.x ? min(kMaxUnits, (units - blockIdx.x + gridDim.x - 1) / gridDim.x) : 0u;
}

// Issues the lane's loads for the tile at the load cursor and advances it; past the wave's
// range it loads the first tile of the matrix instead (an L2 hit, never consumed), so every
// call issues the same number of loads and the compiler can wait for exactly the slot in use.
__device__ __forceinline__ void job_issue(const Job& j, Stream& s, uint32_t lane, Q4Tile& t) {
    const bool real = s.ld.f < s.fe;
    const uint32_t unit = blockIdx.x + s.ld.k * gridDim.x;
    const uint32_t m = j.T == 4 ? s.ld.ts >> 1 : 0u;
    const size_t tile = !real ? 0 : j.T == 4 ? (size_t)unit * 2 + (s.ld.ts & 1) : (size_t)unit;
    const uint4* codes = real && m ? j.codes[1] : j.codes[0];
    const uint2* scales = real && m ? j.scales[1] : j.scales[0];
    q4_tile_load(codes, scales, tile, j.nst, real ? s.ld.st : 0u, lane, t);
    if (real) cur_next(s.ld, j.nst, j.T);
}

// Streaming waves: position the cursors and issue the first kAhead tile loads.
__device__ __forceinline__ void job_prefetch(const Job& j, Stream& s, Q4Tile (&buf)[kAhead], uint32_t wave,
                                             uint32_t lane) {
    const uint32_t F = my_units(j.units) * j.T * j.nst, w = wave - 1;
    const uint32_t fb = (uint32_t)(((uint64_t)F * w) / kStreamWaves);
    s.fe = (uint32_t)(((uint64_t)F * (w + 1)) / kStreamWaves);
    s.ld = cur_at(fb, j.nst, j.T);
    s.cs = s.ld;
#pragma unroll
    for (int u = 0; u < kAhead; ++u) job_issue(j, s, lane, buf[u]);
}

// part[(k * kMaxT + ts) * 8 + wave][16]: one wave's row sums of one tile.  Slot u of the ring
// holds tile fb + u (mod kAhead); each consumed slot is refilled at once.
__device__ __forceinline__ void job_stream(const Job& j, Stream& s, Q4Tile (&buf)[kAhead], const int8_t* dig,
                                           const DigitTab* tab, float* part, uint32_t wave, uint32_t lane) {
    float acc[4] = {0.f, 0.f, 0.f, 0.f};
    const uint32_t n = s.fe - s.cs.f;
    for (uint32_t base = 0; base < n; base += kAhead) {
#pragma unroll
        for (int u = 0; u < kAhead; ++u) {
            if (base + u < n) {
                q4_mfma_tile(buf[u], s.cs.st, dig, tab, lane, acc);
                if (s.cs.st == j.nst - 1 || s.cs.f + 1 == s.fe) {
                    q4_row_sums(acc);
                    if ((lane & 15) == 0) {
                        float* p = part + ((s.cs.k * kMaxT + s.cs.ts) * 8 + wave) * 16 + 4 * (lane >> 4);
#pragma unroll
                        for (int i = 0; i < 4; ++i) p[i] = acc[i];
                    }
#pragma unroll
                    for (int i = 0; i < 4; ++i) acc[i] = 0.0f;
                }
                cur_next(s.cs, j.nst, j.T);
            }
            job_issue(j, s, lane, buf[u]);
        }
    }
}

__device__ __forceinline__ float part_sum(const float* part, uint32_t k, uint32_t ts, uint32_t r) {
    const float* p = part + (k * kMaxT + ts) * 8 * 16 + r;
    float v = p[16];  // wave 0 never streams
#pragma unroll
    for (int w = 2; w < 8; ++w) v += p[16 * w];
    return v;
}

// Input prologue of a GEMV phase: LDS layout [digit image nst * 640][x K][res K][w_a K][w_n K]
// (floats).  Wave 0 stages, every thread then builds the digit image.
enum StageKind { S_EMBED = 0, S_RESID = 1, S_DIGITS = 2 };

struct Stage {
    const float *x, *res, *w_a, *w_n;
    float eps_a, eps_n, scale;
    const int8_t* dig;    // S_DIGITS
    float* x_out;         // S_EMBED / S_RESID: the residual, written by workgroup 0
    float* snap;          // optional copy of x_out
};

__device__ __forceinline__ void stage_inputs(int kind, const Stage& in, uint32_t K, uint32_t nst, uint8_t* lds, uint32_t lane) {
    uint8_t* img = lds;
    float* xs = reinterpret_cast<float*>(lds + (size_t)nst * 640);
    const uint32_t kb = K * 4;
    if (kind == S_DIGITS) {
        dma(in.dig, nst * 640, img, lane);
    } else {
        if (kind == S_RESID) {
            dma(in.x, kb, reinterpret_cast<uint8_t*>(xs), lane);
            dma(in.res, kb, reinterpret_cast<uint8_t*>(xs + K), lane);
            if (in.w_a) dma(in.w_a, kb, reinterpret_cast<uint8_t*>(xs + 2 * K), lane);
        }
        dma(in.w_n, kb, reinterpret_cast<uint8_t*>(xs + 3 * K), lane);
    }
    wait_vm();
}

// Digit image of the normalised input (K <= 4096, so one octet per thread).
__device__ __forceinline__ void stage_digits(int kind, const Stage& in, const InputStage& emb, uint32_t K, uint32_t nst, uint8_t* lds,
                             double* red) {
    int8_t* dig = reinterpret_cast<int8_t*>(lds);
    DigitTab* tab = reinterpret_cast<DigitTab*>(lds + (size_t)nst * 512);
    float* xs = reinterpret_cast<float*>(lds + (size_t)nst * 640);
    const uint32_t tid = threadIdx.x, n8 = K / 8, o = tid;
    const bool ok = o < n8;
    float t[8], v[8];
    if (kind == S_EMBED) {
        embed_row(emb, xs, K);
        __syncthreads();
#pragma unroll
        for (int k = 0; k < 8; ++k) t[k] = ok ? xs[8 * o + k] : 0.0f;
    } else {
        double ra = 1.0;
        if (in.w_a) {
            double sa = 0.0;
            if (ok) {
#pragma unroll
                for (int k = 0; k < 8; ++k) sa += (double)xs[8 * o + k] * xs[8 * o + k];
            }
            ra = inv_rms(block_sum_d(sa, red), K, in.eps_a);
        }
#pragma unroll
        for (int k = 0; k < 8; ++k) {
            if (ok) {
                const float x = xs[8 * o + k], r = xs[K + 8 * o + k];
                const float u = in.w_a ? norm_apply(x, ra, xs[2 * K + 8 * o + k]) : x;
                t[k] = __fmul_rn(__fadd_rn(u, r), in.scale);
            } else {
                t[k] = 0.0f;
            }
        }
    }
    double ss = 0.0;
#pragma unroll
    for (int k = 0; k < 8; ++k) ss += (double)t[k] * t[k];
    if (blockIdx.x == 0 && ok) {
        const v4u a = {__float_as_uint(t[0]), __float_as_uint(t[1]), __float_as_uint(t[2]), __float_as_uint(t[3])};
        const v4u b = {__float_as_uint(t[4]), __float_as_uint(t[5]), __float_as_uint(t[6]), __float_as_uint(t[7])};
        stc16(in.x_out, o * 32, a);
        stc16(in.x_out, o * 32 + 16, b);
        if (in.snap) {
            stc16(in.snap, o * 32, a);
            stc16(in.snap, o * 32 + 16, b);
        }
    }
    const double rn = inv_rms(block_sum_d(ss, red), K, in.eps_n);
#pragma unroll
    for (int k = 0; k < 8; ++k) v[k] = ok ? norm_apply(t[k], rn, xs[3 * K + 8 * o + k]) : 0.0f;
    float m, sum;
    quad_stats(v, m, sum);
    const uint32_t b = o >> 2, p = o & 3;
    if (b < nst * 4) {
        digits8(v, m, dig, b, p);
        if (p == 0) digit_tab(tab, b, m, sum);
    }
}

// Digit image words of one 32-element block held by a quad (8 values per lane), stored
// coherently into the image at block b.
__device__ __forceinline__ void quad_digits_store(const float (&v)[8], int8_t* img, uint32_t nst, uint32_t b,
                                                  uint32_t p) {
    float m, sum;
    quad_stats(v, m, sum);
    uint32_t w[4][2];
    digit_words(v, m, w);
#pragma unroll
    for (int t = 0; t < 4; ++t) stc8(img, (b * 4 + t) * 32 + 8 * p, v2u{w[t][0], w[t][1]});
    if (p == 0) {
        DigitTab e[4];
#pragma unroll
        for (int t = 0; t < 4; ++t) e[t] = digit_entry(m, sum, t);
        const uint32_t base = nst * 512 + b * 32;
        stc16(img, base, v4u{__float_as_uint(e[0].scale), __float_as_uint(e[0].bias), __float_as_uint(e[1].scale),
                             __float_as_uint(e[1].bias)});
        stc16(img, base + 16, v4u{__float_as_uint(e[2].scale), __float_as_uint(e[2].bias),
                                  __float_as_uint(e[3].scale), __float_as_uint(e[3].bias)});
    }
}

// ---- attention phase ------------------------------------------------------------------------------

// Work item (KV head h, chunk c) of the visible range runs on workgroup h * chunks + c with all
// 512 threads; the last chunk of a head to finish merges the head's partials and writes the
// digit image of its query heads' outputs for the o-proj GEMV.
template <int GQ>
__device__ __forceinline__ void attention_item(const StepLayer& L, const StepArgs& a, uint32_t pos, uint32_t h, uint32_t c,
                               uint32_t chunks, uint32_t cmax, uint32_t clen, uint32_t start, uint8_t* lds) {
    constexpr int D = 256, NH = GQ + 2;
    float* nrm = reinterpret_cast<float*>(lds);  // [NH][D]
    float* qs = nrm + NH * D;                     // [GQ][D]
    float* scores = qs + GQ * D;                  // [GQ][kStepMaxClen]
    float* vred = scores + GQ * kStepMaxClen;     // [16][GQ][D]
    double* dred = reinterpret_cast<double*>(vred + 16 * GQ * D);  // [8][NH]
    float* fred = reinterpret_cast<float*>(dred + 8 * NH);         // [8]
    float* cw = fred + 8;                                          // [GQ][kStepMaxChunks] (merge)
    float* cl = cw + GQ * kStepMaxChunks;                          // [GQ][kStepMaxChunks]
    int* flag = reinterpret_cast<int*>(cl + GQ * kStepMaxChunks);

    const uint32_t tid = threadIdx.x, lane = tid & 63, wave = wave_id();
    const uint32_t t0 = start + c * clen, t1 = min(pos + 1, t0 + clen), n = t1 - t0;
    const uint32_t ring = L.ring;
    const bool append = t1 == pos + 1;
    const bool ch = tid < D;

    // prologue: RMSNorm of the query heads (and the new K, V), NeoX RoPE, K/V append
    float raw[NH];
#pragma unroll
    for (int q = 0; q < GQ; ++q) raw[q] = ch ? __uint_as_float(ldc(a.QKV, ((h * GQ + q) * D + tid) * 4)) : 0.0f;
    raw[GQ] = ch && append ? __uint_as_float(ldc(a.QKV, (L.qn + h * D + tid) * 4)) : 0.0f;
    raw[GQ + 1] = ch && append ? __uint_as_float(ldc(a.QKV, (L.v_off + h * D + tid) * 4)) : 0.0f;
    double sn = 0.0, cs = 1.0;
    if (tid < D / 2) sincos((double)pos * gp(L.inv_freq)[tid], &sn, &cs);
#pragma unroll
    for (int q = 0; q < NH; ++q) {
        const double v = wave_sum((double)raw[q] * (double)raw[q]);
        if (lane == 0) dred[wave * NH + q] = v;
    }
    __syncthreads();
    if (ch) {
#pragma unroll
        for (int q = 0; q < NH; ++q) {
            if (q >= GQ && !append) break;
            const double ss = (dred[0 * NH + q] + dred[1 * NH + q]) + (dred[2 * NH + q] + dred[3 * NH + q]);
            float r;
            if (q < GQ) r = norm_apply(raw[q], inv_rms(ss, D, L.q_eps), gp(L.q_norm)[tid]);
            else if (q == GQ) r = norm_apply(raw[q], inv_rms(ss, D, L.k_eps), gp(L.k_norm)[tid]);
            else r = L.v_norm ? (float)__dmul_rn((double)raw[q], inv_rms(ss, D, L.v_eps)) : raw[q];
            nrm[q * D + tid] = r;
        }
    }
    __syncthreads();
    const size_t slot = ((size_t)h * ring + pos % ring) * D;
    if (tid < D / 2) {
#pragma unroll
        for (int q = 0; q < GQ + 1; ++q) {
            if (q == GQ && !append) break;
            const double x = (double)nrm[q * D + tid], y = (double)nrm[q * D + tid + D / 2];
            const float r0 = (float)__dsub_rn(__dmul_rn(x, cs), __dmul_rn(y, sn));
            const float r1 = (float)__dadd_rn(__dmul_rn(x, sn), __dmul_rn(y, cs));
            if (q < GQ) {
                qs[q * D + tid] = r0;
                qs[q * D + tid + D / 2] = r1;
            } else {
                gp(L.kcache)[slot + tid] = f2h(r0);
                gp(L.kcache)[slot + tid + D / 2] = f2h(r1);
            }
        }
    }
    if (append && ch) gp(L.vcache)[slot + tid] = f2h(nrm[(GQ + 1) * D + tid]);
    __syncthreads();

    // scores: 16 lanes per token (16 channels each), 32 token groups
    {
        const uint32_t grp = tid >> 4, j = tid & 15;
        float qr[GQ][16];
#pragma unroll
        for (int q = 0; q < GQ; ++q)
#pragma unroll
            for (int e = 0; e < 16; ++e) qr[q][e] = qs[q * D + 16 * j + e];
        for (uint32_t t = t0 + grp; t < t1; t += 32) {
            const uint16_t* kp = L.kcache + ((size_t)h * ring + t % ring) * D + 16 * j;
            const v4u k0 = *gp(reinterpret_cast<const v4u*>(kp));
            const v4u k1 = *gp(reinterpret_cast<const v4u*>(kp + 8));
            const uint32_t kw[8] = {k0.x, k0.y, k0.z, k0.w, k1.x, k1.y, k1.z, k1.w};
            float kf[16];
#pragma unroll
            for (int e = 0; e < 8; ++e) {
                kf[2 * e] = h2f((uint16_t)(kw[e] & 0xFFFFu));
                kf[2 * e + 1] = h2f((uint16_t)(kw[e] >> 16));
            }
#pragma unroll
            for (int q = 0; q < GQ; ++q) {
                float d = 0.0f;
#pragma unroll
                for (int e = 0; e < 16; ++e) d = fmaf(qr[q][e], kf[e], d);
#pragma unroll
                for (int o = 8; o > 0; o >>= 1) d += __shfl_xor(d, o, 16);
                if (j == 0) scores[q * kStepMaxClen + (t - t0)] = d * L.scale;
            }
        }
    }
    __syncthreads();

    float m[GQ], l[GQ];
#pragma unroll
    for (int q = 0; q < GQ; ++q) {
        float mx = -INFINITY;
        for (uint32_t i = tid; i < n; i += kThreads) mx = fmaxf(mx, scores[q * kStepMaxClen + i]);
        m[q] = block_max_f(mx, fred);
        float sum = 0.0f;
        for (uint32_t i = tid; i < n; i += kThreads) {
            const float p = expf(scores[q * kStepMaxClen + i] - m[q]);
            scores[q * kStepMaxClen + i] = p;
            sum += p;
        }
        l[q] = block_sum_f(sum, fred);
    }
    __syncthreads();

    // values: 32 lanes per token row (8 channels each), 16 token groups
    {
        const uint32_t tg = tid >> 5, dl = tid & 31;
        float acc[GQ][8];
#pragma unroll
        for (int q = 0; q < GQ; ++q)
#pragma unroll
            for (int e = 0; e < 8; ++e) acc[q][e] = 0.0f;
        for (uint32_t t = t0 + tg; t < t1; t += 16) {
            const v4u vv = *gp(reinterpret_cast<const v4u*>(L.vcache + ((size_t)h * ring + t % ring) * D + 8 * dl));
            const uint32_t vw[4] = {vv.x, vv.y, vv.z, vv.w};
            float vf[8];
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                vf[2 * e] = h2f((uint16_t)(vw[e] & 0xFFFFu));
                vf[2 * e + 1] = h2f((uint16_t)(vw[e] >> 16));
            }
#pragma unroll
            for (int q = 0; q < GQ; ++q) {
                const float p = scores[q * kStepMaxClen + (t - t0)];
#pragma unroll
                for (int e = 0; e < 8; ++e) acc[q][e] = fmaf(p, vf[e], acc[q][e]);
            }
        }
#pragma unroll
        for (int q = 0; q < GQ; ++q)
#pragma unroll
            for (int e = 0; e < 8; ++e) vred[(tg * GQ + q) * D + 8 * dl + e] = acc[q][e];
    }
    __syncthreads();

    // chunk partial: o[q][d] (unnormalised), m[q], l[q]
    const uint32_t stride = GQ * (D + 2);
    const uint32_t mine = ((h * cmax + c) * stride) * 4;
    for (uint32_t i = tid; i < GQ * D; i += kThreads) {
        const uint32_t q = i / D, d = i % D;
        float t = 0.0f;
#pragma unroll
        for (int g = 0; g < 16; ++g) t += vred[(g * GQ + q) * D + d];
        stc(a.part, mine + (q * (D + 2) + d) * 4, __float_as_uint(t));
    }
    if (tid < GQ) {
#pragma unroll
        for (int q = 0; q < GQ; ++q) {
            if ((uint32_t)q == tid) {
                stc(a.part, mine + (q * (D + 2) + D) * 4, __float_as_uint(m[q]));
                stc(a.part, mine + (q * (D + 2) + D + 1) * 4, __float_as_uint(l[q]));
            }
        }
    }
    wait_vm();
    __syncthreads();
    if (tid == 0) {
        const uint32_t ticket =
            __hip_atomic_fetch_add(a.counters + h, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        *flag = ticket == chunks - 1;
    }
    __syncthreads();
    if (!*flag) return;

    // merge (last chunk of this head): weights exp(m_c - M), output sum_c w_c o_c / sum_c w_c l_c
    const uint32_t all = (h * cmax * stride) * 4;
    for (uint32_t i = tid; i < chunks * GQ; i += kThreads) {
        const uint32_t k = i / GQ, q = i % GQ;
        cw[q * kStepMaxChunks + k] = __uint_as_float(ldc(a.part, all + (k * stride + q * (D + 2) + D) * 4));
        cl[q * kStepMaxChunks + k] = __uint_as_float(ldc(a.part, all + (k * stride + q * (D + 2) + D + 1) * 4));
    }
    __syncthreads();
    float M[GQ];
#pragma unroll
    for (int q = 0; q < GQ; ++q) {
        M[q] = -INFINITY;
        for (uint32_t k = 0; k < chunks; ++k) M[q] = fmaxf(M[q], cw[q * kStepMaxChunks + k]);
    }
    __syncthreads();
    for (uint32_t i = tid; i < chunks * GQ; i += kThreads) {
        const uint32_t k = i / GQ, q = i % GQ;
        cw[q * kStepMaxChunks + k] = expf(cw[q * kStepMaxChunks + k] - M[q]);
    }
    __syncthreads();
    float* outv = vred;  // [GQ][D]
    for (uint32_t i = tid; i < GQ * D; i += kThreads) {
        const uint32_t q = i / D, d = i % D;
        float Lq = 0.0f, acc = 0.0f;
        for (uint32_t k = 0; k < chunks; ++k) {
            const float w = cw[q * kStepMaxChunks + k];
            Lq = fmaf(w, cl[q * kStepMaxChunks + k], Lq);
            acc = fmaf(w, __uint_as_float(ldc(a.part, all + (k * stride + q * (D + 2) + d) * 4)), acc);
        }
        outv[i] = acc / Lq;
    }
    __syncthreads();
    // digit image blocks (h GQ + q) * 8 + b of the o-proj input: 4 threads per block
    const uint32_t nst_att = L.o.nst;
    if (tid < 32 * GQ) {
        const uint32_t blk = tid >> 2, p = tid & 3;
        float v[8];
#pragma unroll
        for (int k = 0; k < 8; ++k) v[k] = outv[blk * 32 + 8 * p + k];
        quad_digits_store(v, a.att_img, nst_att, h * GQ * 8 + blk, p);
    }
    if (tid == 0) __hip_atomic_store(a.counters + h, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

}  // namespace

// ---- the kernel -----------------------------------------------------------------------------------

template <int GQ>
__global__ __launch_bounds__(512) void decode_step_kernel(StepArgs a) {
    extern __shared__ __align__(16) uint8_t lds[];
    __shared__ float part[kMaxUnits * kMaxT * 8 * 16];
    __shared__ double red[8];
    __shared__ int ok_flag;
    __shared__ float act_l[kMaxUnits][32];

    if (a.state[ST_STOP]) return;  // uniform: written only before the launch
    const uint32_t tid = threadIdx.x, lane = tid & 63, wave = wave_id();
    const uint32_t pos = a.state[ST_POS];
    const uint32_t H = a.hidden, I = a.inter;
    Grid g{a.bar, 0u, &ok_flag, a.clock};
    if (tid == 0) stamp(g, 0);
    bool failed = false;
    Q4Tile buf[kAhead];
    Stream s{};

    auto gemv_job = [&](const Q4View& m0, const Q4View* m1) {
        Job j{};
        j.codes[0] = reinterpret_cast<const uint4*>(m0.codes);
        j.scales[0] = reinterpret_cast<const uint2*>(m0.scales);
        if (m1) {
            j.codes[1] = reinterpret_cast<const uint4*>(m1->codes);
            j.scales[1] = reinterpret_cast<const uint2*>(m1->scales);
            j.units = (m0.rows + 31) / 32;
            j.T = 4;
        } else {
            j.units = (m0.rows + 15) / 16;
            j.T = 1;
        }
        j.nst = m0.nst;
        return j;
    };
    auto zero_part = [&]() {
        for (uint32_t i = tid; i < kMaxUnits * kMaxT * 8 * 16; i += kThreads) part[i] = 0.0f;
    };
    // Streams a GEMV (prefetched already), then leaves its row sums in `part`.
    auto run_stream = [&](const Job& j, uint32_t nst) {
        if (wave != 0) {
            const int8_t* dig = reinterpret_cast<const int8_t*>(lds);
            const DigitTab* tab = reinterpret_cast<const DigitTab*>(lds + (size_t)nst * 512);
            job_stream(j, s, buf, dig, tab, part, wave, lane);
        }
        __syncthreads();
    };

    const uint32_t n_layers = a.n_layers;
    {
        const Job j0 = gemv_job(a.layers[0].qkv, nullptr);
        if (wave != 0) job_prefetch(j0, s, buf, wave, lane);
    }
    for (uint32_t l = 0; l < n_layers; ++l) {
        const StepLayer& L = a.layers[l];
        // ---- qkv: x = embedding (layer 0) or the previous layer's output; y = W_qkv rms(x) w
        {
            if (l > 0 && !grid_sync(g)) {
                failed = true;
                break;
            }
            Stage in{};
            InputStage emb{};
            int kind;
            if (l == 0) {
                kind = S_EMBED;
                emb.table = a.table;
                emb.ids = a.ids;
                emb.state = a.state;
                emb.emb_scale = a.emb_scale;
            } else {
                const StepLayer& P = a.layers[l - 1];
                kind = S_RESID;
                in.x = a.D;
                in.res = a.H;
                in.w_a = P.post_ffn;
                in.eps_a = P.post_ffn_eps;
                in.scale = P.layer_scale;
            }
            in.w_n = L.input_norm;
            in.eps_n = L.input_eps;
            in.x_out = a.X;
            in.snap = a.snap && l > 0 ? a.snap + (size_t)(l - 1) * H : nullptr;
            const Job j = gemv_job(L.qkv, nullptr);
            if (wave == 0) stage_inputs(kind, in, H, j.nst, lds, lane);
            __syncthreads();
            zero_part();
            stage_digits(kind, in, emb, H, j.nst, lds, red);
            __syncthreads();
            run_stream(j, j.nst);
            const uint32_t mu = my_units(j.units);
            if (tid < 16 * mu) {
                const uint32_t k = tid >> 4, r = tid & 15, row = (blockIdx.x + k * gridDim.x) * 16 + r;
                if (row < L.qkv.rows) stc(a.QKV, row * 4, __float_as_uint(part_sum(part, k, 0, r)));
            }
            wait_vm();
        }
        // ---- attention
        {
            if (!grid_sync(g)) {
                failed = true;
                break;
            }
            const uint32_t nvis = L.window ? min(pos + 1, L.window) : pos + 1;
            const uint32_t start = pos + 1 - nvis;
            const uint32_t cmax = a.cmax / L.kv_heads;
            uint32_t chunks = min(cmax, (nvis + kAttnMinChunk - 1) / kAttnMinChunk);
            const uint32_t clen = (nvis + chunks - 1) / chunks;
            chunks = (nvis + clen - 1) / clen;
            const Job jo = gemv_job(L.o, nullptr);
            const uint32_t items = L.kv_heads * chunks;
            if (blockIdx.x < items) {
                attention_item<GQ>(L, a, pos, blockIdx.x / chunks, blockIdx.x % chunks, chunks, cmax, clen, start,
                                   lds);
                wait_vm();
                __syncthreads();
            }
            if (wave != 0) job_prefetch(jo, s, buf, wave, lane);
        }
        // ---- o-proj: input = the attention output's digit image
        {
            if (!grid_sync(g)) {
                failed = true;
                break;
            }
            const Job j = gemv_job(L.o, nullptr);
            Stage in{};
            in.dig = a.att_img;
            if (wave == 0) stage_inputs(S_DIGITS, in, L.o.blocks * 32, j.nst, lds, lane);
            zero_part();
            __syncthreads();
            run_stream(j, j.nst);
            const uint32_t mu = my_units(j.units);
            if (tid < 16 * mu) {
                const uint32_t k = tid >> 4, r = tid & 15, row = (blockIdx.x + k * gridDim.x) * 16 + r;
                if (row < L.o.rows) stc(a.PROJ, row * 4, __float_as_uint(part_sum(part, k, 0, r)));
            }
            wait_vm();
            const Job jg = gemv_job(L.gate, &L.up);
            if (wave != 0) job_prefetch(jg, s, buf, wave, lane);
        }
        // ---- gate/up: x = rms(proj) post_attn + residual; act = gelu(gate) * up, as digits
        {
            if (!grid_sync(g)) {
                failed = true;
                break;
            }
            const Job j = gemv_job(L.gate, &L.up);
            Stage in{};
            InputStage emb{};
            in.x = a.PROJ;
            in.res = a.X;
            in.w_a = L.post_attn;
            in.eps_a = L.post_attn_eps;
            in.scale = 1.0f;
            in.w_n = L.ffn_norm;
            in.eps_n = L.ffn_eps;
            in.x_out = a.H;
            if (wave == 0) stage_inputs(S_RESID, in, H, j.nst, lds, lane);
            __syncthreads();
            zero_part();
            stage_digits(S_RESID, in, emb, H, j.nst, lds, red);
            __syncthreads();
            run_stream(j, j.nst);
            const uint32_t mu = my_units(j.units);
            if (tid < 32 * mu) {
                const uint32_t k = tid >> 5, r = tid & 31, t = r >> 4, rr = r & 15;
                act_l[k][r] = gelu_mul(part_sum(part, k, t, rr), part_sum(part, k, 2 + t, rr));
            }
            __syncthreads();
            if (tid < 4 * mu) {
                const uint32_t k = tid >> 2, p = tid & 3;
                float v[8];
#pragma unroll
                for (int e = 0; e < 8; ++e) v[e] = act_l[k][8 * p + e];
                quad_digits_store(v, a.act_img, L.down.nst, blockIdx.x + k * gridDim.x, p);
            }
            wait_vm();
            const Job jd = gemv_job(L.down, nullptr);
            if (wave != 0) job_prefetch(jd, s, buf, wave, lane);
        }
        // ---- down: input = the activation's digit image
        {
            if (!grid_sync(g)) {
                failed = true;
                break;
            }
            const Job j = gemv_job(L.down, nullptr);
            Stage in{};
            in.dig = a.act_img;
            if (wave == 0) stage_inputs(S_DIGITS, in, I, j.nst, lds, lane);
            zero_part();
            __syncthreads();
            run_stream(j, j.nst);
            const uint32_t mu = my_units(j.units);
            if (tid < 16 * mu) {
                const uint32_t k = tid >> 4, r = tid & 15, row = (blockIdx.x + k * gridDim.x) * 16 + r;
                if (row < L.down.rows) stc(a.D, row * 4, __float_as_uint(part_sum(part, k, 0, r)));
            }
            wait_vm();
            if (l + 1 < n_layers) {
                const Job jn = gemv_job(a.layers[l + 1].qkv, nullptr);
                if (wave != 0) job_prefetch(jn, s, buf, wave, lane);
            }
        }
    }
    grid_exit(g, a.state, a.advance != 0, failed);
}

size_t step_lds_bytes(uint32_t hidden, uint32_t inter, uint32_t q_dim, uint32_t group) {
    const size_t nst_h = (hidden + 127) / 128, nst_i = (inter + 127) / 128, nst_q = (q_dim + 127) / 128;
    size_t g = nst_h * 640 + (size_t)4 * hidden * 4;  // image + staging of a residual prologue
    g = std::max(g, nst_i * 640);
    g = std::max(g, nst_q * 640);
    const size_t D = 256, NH = group + 2;
    const size_t att = 4 * (NH * D + group * D + group * kStepMaxClen + 16 * group * D) + 8 * 8 * NH + 4 * 8 +
                       4 * 2 * group * kStepMaxChunks + 16;
    return std::max(g, att);
}

hipError_t launch_step(const StepArgs& a, uint32_t group, uint32_t grid, size_t lds, hipStream_t s) {
    void* args[] = {const_cast<StepArgs*>(&a)};
    switch (group) {
        case 1: return hipLaunchCooperativeKernel((const void*)decode_step_kernel<1>, dim3(grid), dim3(kThreads), args, lds, s);
        case 2: return hipLaunchCooperativeKernel((const void*)decode_step_kernel<2>, dim3(grid), dim3(kThreads), args, lds, s);
        case 4: return hipLaunchCooperativeKernel((const void*)decode_step_kernel<4>, dim3(grid), dim3(kThreads), args, lds, s);
        default: return hipErrorInvalidValue;
    }
}

hipError_t step_max_grid(uint32_t group, size_t lds, uint32_t* grid) {
    int dev = 0, cus = 0, per = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e == hipSuccess) e = hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev);
    const void* k = group == 1 ? (const void*)decode_step_kernel<1>
                               : group == 2 ? (const void*)decode_step_kernel<2> : (const void*)decode_step_kernel<4>;
    if (e == hipSuccess) e = hipOccupancyMaxActiveBlocksPerMultiprocessor(&per, k, kThreads, lds);
    if (e != hipSuccess) return e;
    *grid = per >= 1 ? (uint32_t)(cus / 8 * 8) : 0u;
    return hipSuccess;
}

}  // namespace af
