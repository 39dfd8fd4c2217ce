// Device helpers shared by the per-operation kernels and the persistent decode-step kernel
// (gfx950): half conversions, wave/block reductions, the reference's fp64 rounding points,
// Q6_K code unpacking, and the Q4_0 GEMV input prologue (int8 digit planes in LDS).
#pragma once
#include <hip/hip_runtime.h>
#include <math.h>

#include "af_internal.h"

namespace af {

// ---- helpers ----------------------------------------------------------------------------------

// Global-address-space views of generic pointers: loads and stores through them are global
// (vector memory counter only) instead of flat (which also counts against the LDS counter).
template <typename T>
__device__ __forceinline__ const __attribute__((address_space(1))) T* gp(const T* p) {
    return (const __attribute__((address_space(1))) T*)p;
}
template <typename T>
__device__ __forceinline__ __attribute__((address_space(1))) T* gp(T* p) {
    return (__attribute__((address_space(1))) T*)p;
}

// The wave's index in its workgroup, known to the compiler as wave-uniform (an SGPR), so that
// control flow derived from it stays scalar.
__device__ __forceinline__ uint32_t wave_id() { return __builtin_amdgcn_readfirstlane(threadIdx.x >> 6); }

__device__ __forceinline__ float h2f(uint16_t b) { return (float)__builtin_bit_cast(_Float16, b); }
__device__ __forceinline__ uint16_t f2h(float f) { return __builtin_bit_cast(uint16_t, (_Float16)f); }

// Cross-lane exchanges on the DPP path (a VALU operand modifier, a few cycles) instead of
// ds_bpermute (an LDS round trip per step).  Controls: quad_perm [1,0,3,2] = lane ^ 1,
// quad_perm [2,3,0,1] = lane ^ 2, row_half_mirror (lane 7 - i within 8), row_mirror (lane
// 15 - i within 16).  Every lane of the 16-lane row must be active.
enum DppCtrl { kDppXor1 = 0xB1, kDppXor2 = 0x4E, kDppHalfMirror = 0x141, kDppMirror = 0x140 };

template <int C>
__device__ __forceinline__ float dpp(float v) {
    return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), C, 0xF, 0xF, false));
}
template <int C>
__device__ __forceinline__ double dpp(double v) {
    const uint64_t u = __builtin_bit_cast(uint64_t, v);
    const uint32_t lo = (uint32_t)__builtin_amdgcn_update_dpp(0, (int)(uint32_t)u, C, 0xF, 0xF, false);
    const uint32_t hi = (uint32_t)__builtin_amdgcn_update_dpp(0, (int)(uint32_t)(u >> 32), C, 0xF, 0xF, false);
    return __builtin_bit_cast(double, ((uint64_t)hi << 32) | lo);
}

// Sum (max) over each 16-lane row, left in every lane of the row.  After the two quad steps
// every lane of a quad holds the quad's value, so mirroring pairs each lane with the other
// quad (half row), then with the other half row.
template <typename T>
__device__ __forceinline__ T row_sum(T v) {
    v += dpp<kDppXor1>(v);
    v += dpp<kDppXor2>(v);
    v += dpp<kDppHalfMirror>(v);
    v += dpp<kDppMirror>(v);
    return v;
}
__device__ __forceinline__ float row_max(float v) {
    v = fmaxf(v, dpp<kDppXor1>(v));
    v = fmaxf(v, dpp<kDppXor2>(v));
    v = fmaxf(v, dpp<kDppHalfMirror>(v));
    v = fmaxf(v, dpp<kDppMirror>(v));
    return v;
}

__device__ __forceinline__ float lane_value(float v, int l) {
    return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), l));
}
__device__ __forceinline__ double lane_value(double v, int l) {
    const uint64_t u = __builtin_bit_cast(uint64_t, v);
    const uint32_t lo = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)u, l);
    const uint32_t hi = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)(u >> 32), l);
    return __builtin_bit_cast(double, ((uint64_t)hi << 32) | lo);
}

// Sum (max) over the wave (all 64 lanes active), the same value in every lane.
template <typename T>
__device__ __forceinline__ T wave_sum(T v) {
    v = row_sum(v);
    return (lane_value(v, 0) + lane_value(v, 16)) + (lane_value(v, 32) + lane_value(v, 48));
}

__device__ __forceinline__ float wave_max(float v) {
    v = row_max(v);
    return fmaxf(fmaxf(lane_value(v, 0), lane_value(v, 16)), fmaxf(lane_value(v, 32), lane_value(v, 48)));
}

// Sum over a 512-thread block of one double per thread, with one barrier: red holds 8 slots used
// by this call alone (a second call needs other slots, or a barrier in between).
__device__ inline double block_sum_once(double v, double* red) {
    v = wave_sum(v);
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = v;
    __syncthreads();
    return ((red[0] + red[1]) + (red[2] + red[3])) + ((red[4] + red[5]) + (red[6] + red[7]));
}

// Sum over the block of one double per thread (blockDim a multiple of 64, <= 512).
__device__ inline double block_sum_d(double v, double* red) {
    v = wave_sum(v);
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, nw = blockDim.x >> 6;
    __syncthreads();
    if (lane == 0) red[wave] = v;
    __syncthreads();
    double t = 0.0;
    for (int w = 0; w < nw; ++w) t += red[w];
    return t;
}

__device__ inline float block_sum_f(float v, float* red) {
    v = wave_sum(v);
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, nw = blockDim.x >> 6;
    __syncthreads();
    if (lane == 0) red[wave] = v;
    __syncthreads();
    float t = 0.0f;
    for (int w = 0; w < nw; ++w) t += red[w];
    return t;
}

__device__ inline float block_max_f(float v, float* red) {
    v = wave_max(v);
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, nw = blockDim.x >> 6;
    __syncthreads();
    if (lane == 0) red[wave] = v;
    __syncthreads();
    float t = red[0];
    for (int w = 1; w < nw; ++w) t = fmaxf(t, red[w]);
    return t;
}

// Sum over the four lanes of a row (l % 16 equal), left in every lane: the 32-lane halves, then
// the 16-lane rows, swapped in registers (v_permlane32_swap / v_permlane16_swap).
__device__ __forceinline__ float row_total(float v) {
    const auto h = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    const float w = __uint_as_float(h[0]) + __uint_as_float(h[1]);
    const auto q = __builtin_amdgcn_permlane16_swap(__float_as_uint(w), __float_as_uint(w), false, false);
    return __uint_as_float(q[0]) + __uint_as_float(q[1]);
}

// f32(x * r * w) with the products in double, as the FP64 RMSNorm oracle rounds its output.
__device__ __forceinline__ float norm_apply(float x, double r, float w) {
    return (float)__dmul_rn(__dmul_rn((double)x, r), (double)w);
}

__device__ __forceinline__ double inv_rms(double sumsq, uint32_t n, float eps) {
    return 1.0 / sqrt(__dadd_rn(sumsq / (double)n, (double)eps));
}

// 1 / sqrt(sumsq / n + eps) from the hardware estimate and two Newton steps
// y <- y (1.5 - 0.5 x y^2): each step roughly doubles the correct bits of the ~2^-22-accurate
// estimate, so the result is within a few double ulps of the division and square root above
// (the f32 values it scales round identically but in rare ties).
__device__ __forceinline__ double inv_rms_fast(double sumsq, uint32_t n, float eps) {
    const double x = __dadd_rn(sumsq / (double)n, (double)eps);
    double y = __builtin_amdgcn_rsq(x);
    y = y * __fma_rn(-0.5 * x * y, y, 1.5);
    y = y * __fma_rn(-0.5 * x * y, y, 1.5);
    return y;
}

// 0.5 x (1 + tanh(sqrt(2/pi) (x + 0.044715 x^3))) in double, rounded to f32, times up in f32.
__device__ __forceinline__ float gelu_mul(float g, float u) {
    const double x = (double)g;
    const double c = sqrt(2.0 / 3.14159265358979323846);
    const double inner = __dadd_rn(x, __dmul_rn(__dmul_rn(__dmul_rn(0.044715, x), x), x));
    const double t = tanh(__dmul_rn(c, inner));
    const float gl = (float)__dmul_rn(__dmul_rn(0.5, x), __dadd_rn(1.0, t));
    return __fmul_rn(gl, u);
}

// One 64-weight Q6_K unit's code bytes for quarter q from its ql/ql/qh dwords.
__device__ __forceinline__ uint32_t q6_codes(uint32_t a, uint32_t b, uint32_t h, int q) {
    switch (q) {
        case 0: return (a & 0x0F0F0F0Fu) | ((h << 4) & 0x30303030u);
        case 1: return (b & 0x0F0F0F0Fu) | ((h << 2) & 0x30303030u);
        case 2: return ((a >> 4) & 0x0F0F0F0Fu) | (h & 0x30303030u);
        default: return ((b >> 4) & 0x0F0F0F0Fu) | ((h >> 2) & 0x30303030u);
    }
}

// ---- input stage: builds the fp32 GEMV input vector in LDS ------------------------------------

// Embedding row (Q6_K, repacked) times emb_scale into xs; one thread per unit dword (16
// elements), threads first, first + step, ... of the caller's range.
// Table row `row`, dequantised and times emb_scale, into xs (elements first, first + step, ...).
__device__ inline void embed_row_at(const Q6View& t, uint32_t row, float emb_scale, float* xs, uint32_t first,
                                    uint32_t step) {
    row = min(row, t.rows - 1);  // ids are validated; never read past the table
    const uint32_t units = t.units, sblocks = units / 4;
    const auto* A = gp(reinterpret_cast<const uint32_t*>(t.a + (size_t)row * units * 16));
    const auto* B = gp(reinterpret_cast<const uint32_t*>(t.b + (size_t)row * units * 16));
    const auto* H = gp(reinterpret_cast<const uint32_t*>(t.h + (size_t)row * units * 16));
    for (uint32_t w = first; w < units * 4; w += step) {
        const uint32_t u = w >> 2, k = w & 3;
        const uint32_t sb = u >> 2, g = (u >> 1) & 1, hh = u & 1;
        const uint32_t a = A[w], b = B[w], h = H[w];
        const uint32_t sc = gp(t.s)[(size_t)row * units + u];
        const float d = h2f(gp(t.d)[(size_t)row * sblocks + sb]);
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            const uint32_t c = q6_codes(a, b, h, q);
            const float ds = __fmul_rn(d, (float)(int8_t)(sc >> (8 * q)));
#pragma unroll
            for (int n = 0; n < 4; ++n) {
                const int code = (int)((c >> (8 * n)) & 0xFF) - 32;
                const uint32_t e = sb * 256 + g * 128 + q * 32 + hh * 16 + 4 * k + n;
                xs[e] = __fmul_rn(__fmul_rn(ds, (float)code), emb_scale);
            }
        }
    }
}

// The row of the token at the session position (ids[state[ST_POS]]).
__device__ inline void embed_row(const InputStage& in, float* xs, uint32_t first, uint32_t step) {
    embed_row_at(in.table, gp(in.ids)[gp(in.state)[ST_POS]], in.emb_scale, xs, first, step);
}

// Loads N float4 per thread from p at float4 indices base + j * blockDim + thread (zero past n4).
// All loads are issued before any is used, so one memory latency covers the whole batch.
template <int N>
__device__ __forceinline__ void load_f4(const float* __restrict__ p, uint32_t base, uint32_t n4, float4 (&o)[N]) {
#pragma unroll
    for (int j = 0; j < N; ++j) {
        const uint32_t i = base + j * blockDim.x + threadIdx.x;
        o[j] = i < n4 ? reinterpret_cast<const float4*>(p)[i] : make_float4(0.f, 0.f, 0.f, 0.f);
    }
}

__device__ __forceinline__ double sq4(float4 v) {
    return (double)v.x * v.x + (double)v.y * v.y + (double)v.z * v.z + (double)v.w * v.w;
}

__device__ __forceinline__ float4 norm4(float4 x, double r, float4 w) {
    return make_float4(norm_apply(x.x, r, w.x), norm_apply(x.y, r, w.y), norm_apply(x.z, r, w.z),
                       norm_apply(x.w, r, w.w));
}

__device__ __forceinline__ float4 resid4(float4 t, float4 res, float scale) {
    return make_float4(__fmul_rn(__fadd_rn(t.x, res.x), scale), __fmul_rn(__fadd_rn(t.y, res.y), scale),
                       __fmul_rn(__fadd_rn(t.z, res.z), scale), __fmul_rn(__fadd_rn(t.w, res.w), scale));
}

// Builds the normalised fp32 input vector in LDS (IN_NORM, IN_RESID, IN_EMBED).  K % 4 == 0 and
// every vector is 16-byte aligned.  Passes cover 4 float4 per thread (4096 floats at 256
// threads), so for the model widths each loop body runs once with its loads batched.
template <int IN>
__device__ inline void input_stage(const InputStage& in, float* xs, uint32_t K, double* red) {
    constexpr int PER = 4;
    const uint32_t tid = threadIdx.x, K4 = K / 4, span = PER * blockDim.x;
    float4* xs4 = reinterpret_cast<float4*>(xs);
    const bool writer = blockIdx.x == 0 && in.x_out != nullptr;
    double ss = 0.0;
    if constexpr (IN == IN_NORM) {
        for (uint32_t b = 0; b < K4; b += span) {
            float4 v[PER];
            load_f4(in.x, b, K4, v);
#pragma unroll
            for (int j = 0; j < PER; ++j) {
                const uint32_t i = b + j * blockDim.x + tid;
                if (i < K4) {
                    xs4[i] = v[j];
                    ss += sq4(v[j]);
                }
            }
        }
    } else if constexpr (IN == IN_RESID) {
        double ra = 1.0;
        if (in.w_a) {
            double sa = 0.0;
            for (uint32_t b = 0; b < K4; b += span) {
                float4 v[PER];
                load_f4(in.x, b, K4, v);
#pragma unroll
                for (int j = 0; j < PER; ++j) sa += sq4(v[j]);
            }
            ra = inv_rms(block_sum_d(sa, red), K, in.eps_a);
        }
        for (uint32_t b = 0; b < K4; b += span) {
            float4 x[PER], r[PER], w[PER];
            load_f4(in.x, b, K4, x);
            load_f4(in.res, b, K4, r);
            if (in.w_a) load_f4(in.w_a, b, K4, w);
#pragma unroll
            for (int j = 0; j < PER; ++j) {
                const uint32_t i = b + j * blockDim.x + tid;
                if (i < K4) {
                    const float4 t = in.w_a ? norm4(x[j], ra, w[j]) : x[j];
                    const float4 v = resid4(t, r[j], in.scale);
                    xs4[i] = v;
                    ss += sq4(v);
                    if (writer) reinterpret_cast<float4*>(in.x_out)[i] = v;
                }
            }
        }
    } else {  // IN_EMBED
        embed_row(in, xs, threadIdx.x, blockDim.x);
        __syncthreads();
        for (uint32_t i = tid; i < K4; i += blockDim.x) {
            const float4 v = xs4[i];
            ss += sq4(v);
            if (writer) reinterpret_cast<float4*>(in.x_out)[i] = v;
        }
    }
    const double rn = inv_rms(block_sum_d(ss, red), K, in.eps_n);
    for (uint32_t b = 0; b < K4; b += span) {
        float4 w[PER];
        load_f4(in.w_n, b, K4, w);
#pragma unroll
        for (int j = 0; j < PER; ++j) {
            const uint32_t i = b + j * blockDim.x + tid;
            if (i < K4) xs4[i] = norm4(xs4[i], rn, w[j]);
        }
    }
    __syncthreads();
}

// ---- Q4_0 GEMV on the int8 matrix cores ---------------------------------------------------------
//
// y = W x with W in Q4_0 and x fp32.  Each 32-element block b of x is written as
//   x_j ~ s_b (q0_j + q1_j 2^-7 + q2_j 2^-14 + q3_j 2^-21),  s_b = 2^(e - 5),  e = ilogb(max |x_b|),
// with integer digits |q| <= 64: elements with |x_j| >= 2^(e - 3) exactly, the others rounded to
// the grid 2^(e - 26), an error of at most 2^(e - 27) <= 2^-27 max |x_b| (digit_words).  Then for
// row r and block b
//   sum_j (n_rj - 8) x_j = sum_t 2^-7t s_b sum_j n_rj q_tj  -  8 sum_j x_j,
// and the integer sums over j come from v_mfma_i32_16x16x64_i8: A = the raw nibbles n of a
// 16-row tile (lane (r, g) holds block g of row r: low nibbles feed one MFMA, high nibbles a
// second), B = the digits, with MFMA column n = (block n / 4, digit n % 4), so both MFMAs of
// a 128-column super-tile accumulate into one 16 x 16 int32 tile.  Lanes then fold the tile
// into fp32 row partials with the block scales d, reduce over the 16 columns, and the waves
// that split the super-tiles of a row tile add their partials in LDS in slice order.

typedef int v4i __attribute__((ext_vector_type(4)));
typedef unsigned v4u __attribute__((ext_vector_type(4)));
typedef float v4f __attribute__((ext_vector_type(4)));

// LDS access by 32-bit byte address (ds_* with a VGPR address and no 64-bit arithmetic).
typedef __attribute__((address_space(3))) uint8_t lds_u8;
template <typename T>
__device__ __forceinline__ T lds_at(uint32_t addr) {
    return *reinterpret_cast<const __attribute__((address_space(3))) T*>(static_cast<uintptr_t>(addr));
}
__device__ __forceinline__ uint32_t lds_addr(const void* p) {
    return (uint32_t)reinterpret_cast<uintptr_t>((const lds_u8*)p);
}
typedef unsigned v2u __attribute__((ext_vector_type(2)));

// Streaming loads of weights (read once per step): non-temporal hint, global address space
// (a generic pointer would become a flat load, which also counts against the LDS counter).
typedef const __attribute__((address_space(1))) v4u* gv4u;
typedef const __attribute__((address_space(1))) v2u* gv2u;
__device__ __forceinline__ uint4 ld_stream(const uint4* p) {
    const v4u t = __builtin_nontemporal_load((gv4u)(p));
    return make_uint4(t.x, t.y, t.z, t.w);
}
__device__ __forceinline__ uint2 ld_stream(const uint2* p) {
    const v2u t = __builtin_nontemporal_load((gv2u)(p));
    return make_uint2(t.x, t.y);
}

// Digit words of 8 consecutive elements v of a block whose max |x| is m: w[t] holds the 8
// int8 digits of plane t.  With s = 2^(ilogb(m) - 5), U = rint(v 2^21 / s) is an integer with
// |U| <= 2^27 (|v| < 2^(ilogb(m) + 1), and scaling by a power of two is exact), and its signed
// radix-2^7 digits satisfy U = 2^21 q0 + 2^14 q1 + 2^7 q2 + q3, so v = s (q0 + q1 2^-7 + q2 2^-14
// + q3 2^-21) to within half of s 2^-21.  The digits are signed 7-bit fields: q3 = sext(U[0, 7)),
// so U - q3 = 2^7 floor((U + 64) / 2^7); q2 = sext((U + 64)[7, 14)); q1 = sext((U + 8256)[14, 21));
// q0 = floor((U + 1056832) / 2^21), with 8256 = 64 (1 + 2^7) and 1056832 = 64 (1 + 2^7 + 2^14).
// q1..q3 lie in [-64, 63] and q0 in [-64, 64].  One bitfield extract (and one add) per digit,
// then v_perm packs the low bytes.
__device__ __forceinline__ uint32_t pack4(int a, int b, int c, int d) {
    // byte i of the result = low byte of the i-th argument
    const uint32_t lo = __builtin_amdgcn_perm((uint32_t)b, (uint32_t)a, 0x0C0C0400u);  // [a0, b0, 0, 0]
    const uint32_t hi = __builtin_amdgcn_perm((uint32_t)d, (uint32_t)c, 0x0C0C0400u);  // [c0, d0, 0, 0]
    return __builtin_amdgcn_perm(hi, lo, 0x05040100u);                                 // [a0, b0, c0, d0]
}

__device__ __forceinline__ void digit_words(const float (&v)[8], float m, uint32_t (&w)[4][2]) {
    const int e = m > 0.0f ? ilogbf(m) : 0;
    int q[4][8];
#pragma unroll
    for (int k = 0; k < 8; ++k) {
        const int U = m > 0.0f ? (int)rintf(ldexpf(v[k], 26 - e)) : 0;
        q[0][k] = (U + 1056832) >> 21;
        q[1][k] = __builtin_amdgcn_sbfe(U + 8256, 14, 7);
        q[2][k] = __builtin_amdgcn_sbfe(U + 64, 7, 7);
        q[3][k] = __builtin_amdgcn_sbfe(U, 0, 7);
    }
#pragma unroll
    for (int t = 0; t < 4; ++t) {
        w[t][0] = pack4(q[t][0], q[t][1], q[t][2], q[t][3]);
        w[t][1] = pack4(q[t][4], q[t][5], q[t][6], q[t][7]);
    }
}

// Digits of 8 consecutive elements v of block b (part p of 4), stored at dig[(b * 4 + t) * 32 + 8 p].
__device__ __forceinline__ void digits8(const float (&v)[8], float m, int8_t* dig, uint32_t b, uint32_t p) {
    uint32_t w[4][2];
    digit_words(v, m, w);
    // plane (i + b) % 4 at store i: the 16 blocks of a wave spread over four LDS bank groups
    // instead of all starting at bank 0 (blocks are 128 bytes apart)
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const uint32_t t = (i + b) & 3;
        uint32_t lo = w[0][0], hi = w[0][1];
        lo = t == 1 ? w[1][0] : lo;
        hi = t == 1 ? w[1][1] : hi;
        lo = t == 2 ? w[2][0] : lo;
        hi = t == 2 ? w[2][1] : hi;
        lo = t == 3 ? w[3][0] : lo;
        hi = t == 3 ? w[3][1] : hi;
        *reinterpret_cast<uint2*>(dig + ((size_t)b * 4 + t) * 32 + 8 * p) = make_uint2(lo, hi);
    }
}

// Block max |x| and sum over the 4 lanes (a quad) that hold a block's 8-element parts.
__device__ __forceinline__ void quad_stats(const float (&v)[8], float& m, float& sum) {
    float mm = 0.0f, ss = 0.0f;
#pragma unroll
    for (int k = 0; k < 8; ++k) {
        mm = fmaxf(mm, fabsf(v[k]));
        ss += v[k];
    }
    mm = fmaxf(mm, dpp<kDppXor1>(mm));
    mm = fmaxf(mm, dpp<kDppXor2>(mm));
    ss += dpp<kDppXor1>(ss);
    ss += dpp<kDppXor2>(ss);
    m = mm;
    sum = ss;
}

// Table entries of a block (max |x| m, element sum `sum`): plane scales s 2^-7t and the bias.
// The table entry of a block of max |x| m and element sum `sum` (BlockTab).
__device__ __forceinline__ BlockTab block_tab(float m, float sum) {
    const float s = m > 0.0f ? ldexpf(1.0f, ilogbf(m) - 5) : 0.0f;
    return BlockTab{ldexpf(s, -14), ldexpf(s, -21), -8.0f * sum, 0.0f};
}

// ---- GEMV prologue: the input's digit image in LDS ----------------------------------------------
//
// Thread i takes the octets (8 consecutive elements) o = i + j * blockDim, j < Q, so the four
// threads of a quad hold one 32-element block.  The kernel issues these input loads before its
// weight loads: vector memory loads return in issue order, so input loads queued behind the
// weight stream would wait for all of it, while issued first they return early and the
// prologue's arithmetic runs while the weights stream in.

template <int IN, int Q>
struct InputRegs {
    float4 x[Q][2], r[Q][2], wa[Q][2], wn[Q][2];
    uint4 d[3 * Q];  // IN_DIGITS: the digit image, 16 bytes per thread and slot
};

__device__ __forceinline__ void ld_oct(const float* p, uint32_t o, bool ok, float4 (&v)[2]) {
    const float4* q = reinterpret_cast<const float4*>(p) + 2 * (size_t)(ok ? o : 0);
    v[0] = ok ? q[0] : make_float4(0.f, 0.f, 0.f, 0.f);
    v[1] = ok ? q[1] : make_float4(0.f, 0.f, 0.f, 0.f);
}

__device__ __forceinline__ void oct_f(const float4 (&v)[2], float (&o)[8]) {
    o[0] = v[0].x; o[1] = v[0].y; o[2] = v[0].z; o[3] = v[0].w;
    o[4] = v[1].x; o[5] = v[1].y; o[6] = v[1].z; o[7] = v[1].w;
}

// Issues every global load the prologue needs (no use of the results).
template <int IN, int Q>
__device__ __forceinline__ void input_load(const InputStage& in, uint32_t K, uint32_t nst, InputRegs<IN, Q>& g) {
    const uint32_t tid = threadIdx.x;
    if constexpr (IN == IN_DIGITS) {
        const uint4* src = reinterpret_cast<const uint4*>(in.dig);
        const uint32_t n16 = nst * (kStepImg / 16);
#pragma unroll
        for (int j = 0; j < 3 * Q; ++j) {
            const uint32_t i = tid + j * blockDim.x;
            g.d[j] = i < n16 ? src[i] : make_uint4(0u, 0u, 0u, 0u);
        }
    } else {
        const uint32_t n8 = K / 8;
#pragma unroll
        for (int j = 0; j < Q; ++j) {
            const uint32_t o = tid + j * blockDim.x;
            const bool ok = o < n8;
            if constexpr (IN != IN_EMBED) ld_oct(in.x, o, ok, g.x[j]);
            if constexpr (IN == IN_RESID) {
                ld_oct(in.res, o, ok, g.r[j]);
                if (in.w_a) ld_oct(in.w_a, o, ok, g.wa[j]);
            }
            if constexpr (IN != IN_PLAIN) ld_oct(in.w_n, o, ok, g.wn[j]);
        }
    }
}

// Finishes the prologue from the registers input_load filled: the LDS digit image of the input.
// xs (K floats of LDS) is used by IN_EMBED only.  The caller syncs.  An input with an RMSNorm
// (IN_NORM, IN_RESID, IN_EMBED), f32(t rn w_n) with rn = rms(t)^-1, is imaged as u = f32(t w_n),
// and the kernel scales its row sums by rn (gemv_row_factor), so the image does not wait for the
// block sum of squares of t; its wave sums are left in red[8, 16).  (The difference is the f32
// rounding of each input element, about 2^-24 of it.)  red: 16 slots.
template <int IN, int Q>
__device__ inline void input_digits(const InputStage& in, uint32_t K, uint32_t nst, InputRegs<IN, Q>& g, float* xs,
                             int8_t* dig, BlockTab* tab, double* red) {
    const uint32_t tid = threadIdx.x, n8 = K / 8;
    if constexpr (IN == IN_DIGITS) {
        uint4* dst = reinterpret_cast<uint4*>(dig);  // digits and table are contiguous
#pragma unroll
        for (int j = 0; j < 3 * Q; ++j) {
            const uint32_t i = tid + j * blockDim.x;
            if (i < nst * (kStepImg / 16)) dst[i] = g.d[j];
        }
        return;
    } else {
        float v[Q][8];
        if constexpr (IN == IN_PLAIN) {
#pragma unroll
            for (int j = 0; j < Q; ++j) oct_f(g.x[j], v[j]);
        } else {
            float t[Q][8];
            if constexpr (IN == IN_EMBED) {
                embed_row(in, xs, threadIdx.x, blockDim.x);
                __syncthreads();
#pragma unroll
                for (int j = 0; j < Q; ++j) {
                    const uint32_t o = tid + j * blockDim.x;
                    float4 e[2];
                    if (o < n8) {
                        e[0] = reinterpret_cast<const float4*>(xs)[2 * o];
                        e[1] = reinterpret_cast<const float4*>(xs)[2 * o + 1];
                    } else {
                        e[0] = e[1] = make_float4(0.f, 0.f, 0.f, 0.f);
                    }
                    oct_f(e, t[j]);
                }
            } else if constexpr (IN == IN_NORM) {
#pragma unroll
                for (int j = 0; j < Q; ++j) oct_f(g.x[j], t[j]);
            } else {  // IN_RESID: t = ((w_a ? rms(x) w_a : x) + res) * scale
                double ra = 1.0;
                if (in.w_a) {
                    double sa = 0.0;
#pragma unroll
                    for (int j = 0; j < Q; ++j) sa += sq4(g.x[j][0]) + sq4(g.x[j][1]);
                    ra = inv_rms_fast(block_sum_once(sa, red), K, in.eps_a);
                }
#pragma unroll
                for (int j = 0; j < Q; ++j) {
#pragma unroll
                    for (int h = 0; h < 2; ++h) {
                        const float4 u = in.w_a ? norm4(g.x[j][h], ra, g.wa[j][h]) : g.x[j][h];
                        g.x[j][h] = resid4(u, g.r[j][h], in.scale);
                    }
                    oct_f(g.x[j], t[j]);
                }
            }
            double ss = 0.0;
#pragma unroll
            for (int j = 0; j < Q; ++j)
#pragma unroll
                for (int k = 0; k < 8; ++k) ss += (double)t[j][k] * t[j][k];
            if (IN != IN_NORM && blockIdx.x == 0 && in.x_out != nullptr) {
#pragma unroll
                for (int j = 0; j < Q; ++j) {
                    const uint32_t o = tid + j * blockDim.x;
                    if (o < n8) {
                        float4* dst = reinterpret_cast<float4*>(in.x_out) + 2 * (size_t)o;
                        dst[0] = make_float4(t[j][0], t[j][1], t[j][2], t[j][3]);
                        dst[1] = make_float4(t[j][4], t[j][5], t[j][6], t[j][7]);
                    }
                }
            }
            ss = wave_sum(ss);
            if ((tid & 63) == 0) red[8 + (tid >> 6)] = ss;
#pragma unroll
            for (int j = 0; j < Q; ++j) {
                float w[8];
                oct_f(g.wn[j], w);
#pragma unroll
                for (int k = 0; k < 8; ++k) v[j][k] = __fmul_rn(t[j][k], w[k]);
            }
        }
#pragma unroll
        for (int j = 0; j < Q; ++j) {
            const uint32_t o = tid + j * blockDim.x, b = o >> 2, p = o & 3;
            float m, sum;
            quad_stats(v[j], m, sum);  // every lane of the quad takes part, in range or not
            if (b < nst * 4) {
                digits8(v[j], m, dig, b, p);
                if (p == 0) tab[b] = block_tab(m, sum);
            }
        }
    }
}

// The RMSNorm row factor rn of a GEMV whose input_digits left the wave sums of squares in
// red[8, 16) (1 for an input without a norm); after a barrier that follows input_digits.
template <int IN>
__device__ __forceinline__ double gemv_row_factor(const double* red, uint32_t K, float eps) {
    if constexpr (IN == IN_NORM || IN == IN_RESID || IN == IN_EMBED) {
        const double ss = ((red[8] + red[9]) + (red[10] + red[11])) + ((red[12] + red[13]) + (red[14] + red[15]));
        return inv_rms_fast(ss, K, eps);
    } else {
        return 1.0;
    }
}

struct Q4Tile {
    uint4 code;      // lane 16 g + r: the 16 code bytes of block g of row r of the super-tile
    uint32_t scale;  // lane 16 g + r: the fp16 scale of block g of row r (low half)
};

// acc += row r's part of one record (super-tile st of a 16-row tile) times the input, for lane
// 16 q + r: two int8 MFMAs with A = the digit planes (row m = 4 g + t: digit t of block g, non-zero
// in k-group g only; a0 / a1 the lane's plane or the zero block, chosen by the caller's address)
// and B = the codes (low nibbles against elements 0..15, high nibbles against 16..31), so the lane
// receives D[4 q + t][r], the digit sums of block q and row r, and adds
// d(r, q) ((2^14 D0 + 2^7 D1 + D2) s 2^-14 + D3 s 2^-21 - 8 sum_j x_j).  2^14 D0 + 2^7 D1 + D2 is
// exact in int32 (|D_t| <= 32 * 15 * 64).
__device__ __forceinline__ void q4_mfma_tile(const Q4Tile& w, const v4i& a0, const v4i& a1, const BlockTab& tb,
                                             float& acc) {
    constexpr uint32_t M = 0x0F0F0F0Fu;
    const uint4 c = w.code;
    const v4i bl = {(int)(c.x & M), (int)(c.y & M), (int)(c.z & M), (int)(c.w & M)};
    const v4i bh = {(int)((c.x >> 4) & M), (int)((c.y >> 4) & M), (int)((c.z >> 4) & M), (int)((c.w >> 4) & M)};
    const v4i zero = {0, 0, 0, 0};
    v4i d = __builtin_amdgcn_mfma_i32_16x16x64_i8(a0, bl, zero, 0, 0, 0);
    d = __builtin_amdgcn_mfma_i32_16x16x64_i8(a1, bh, d, 0, 0, 0);
    const int I = (d[0] << 14) + (d[1] << 7) + d[2];
    float in = fmaf((float)I, tb.s14, tb.nbias);
    in = fmaf((float)d[3], tb.s21, in);
    acc = fmaf(h2f((uint16_t)w.scale), in, acc);
}


}  // namespace af
