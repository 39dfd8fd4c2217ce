// HIP kernels for gfx950 (MI355X): the batch-1 decode step of a Q4_0 / Q6_K
// transformer.  Every kernel is bandwidth-bound GEMV or streaming work; none
// uses MFMA.  Cross-workgroup results (attention chunks, argmax partials) are
// combined by the last workgroup to finish, found with a device-scope counter
// that the last workgroup resets, so the kernels can be replayed in a graph.
#include <hip/hip_runtime.h>
#include <math.h>

#include "af_internal.h"

namespace af {

// ---- helpers ----------------------------------------------------------------------------------

__device__ __forceinline__ float h2f(uint16_t b) { return (float)__builtin_bit_cast(_Float16, b); }
__device__ __forceinline__ uint16_t f2h(float f) { return __builtin_bit_cast(uint16_t, (_Float16)f); }

template <typename T>
__device__ __forceinline__ T wave_sum(T v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
    return v;
}

__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, 64));
    return v;
}

// Sum over the block of one double per thread (blockDim a multiple of 64, <= 512).
__device__ double block_sum_d(double v, double* red) {
    v = wave_sum(v);
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, nw = blockDim.x >> 6;
    __syncthreads();
    if (lane == 0) red[wave] = v;
    __syncthreads();
    double t = 0.0;
    for (int w = 0; w < nw; ++w) t += red[w];
    return t;
}

__device__ float block_sum_f(float v, float* red) {
    v = wave_sum(v);
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, nw = blockDim.x >> 6;
    __syncthreads();
    if (lane == 0) red[wave] = v;
    __syncthreads();
    float t = 0.0f;
    for (int w = 0; w < nw; ++w) t += red[w];
    return t;
}

__device__ float block_max_f(float v, float* red) {
    v = wave_max(v);
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, nw = blockDim.x >> 6;
    __syncthreads();
    if (lane == 0) red[wave] = v;
    __syncthreads();
    float t = red[0];
    for (int w = 1; w < nw; ++w) t = fmaxf(t, red[w]);
    return t;
}

// f32(x * r * w) with the products in double, as the FP64 RMSNorm oracle rounds its output.
__device__ __forceinline__ float norm_apply(float x, double r, float w) {
    return (float)__dmul_rn(__dmul_rn((double)x, r), (double)w);
}

__device__ __forceinline__ double inv_rms(double sumsq, uint32_t n, float eps) {
    return 1.0 / sqrt(__dadd_rn(sumsq / (double)n, (double)eps));
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

// Embedding row (Q6_K, repacked) times emb_scale into xs; one thread per unit dword (16 elements).
__device__ void embed_row(const InputStage& in, float* xs, uint32_t K) {
    const Q6View& t = in.table;
    const uint32_t row = min(in.ids[in.state[ST_POS]], t.rows - 1);  // ids are validated; never read past the table
    const uint32_t units = t.units, sblocks = units / 4;
    const uint32_t* A = reinterpret_cast<const uint32_t*>(t.a + (size_t)row * units * 16);
    const uint32_t* B = reinterpret_cast<const uint32_t*>(t.b + (size_t)row * units * 16);
    const uint32_t* H = reinterpret_cast<const uint32_t*>(t.h + (size_t)row * units * 16);
    for (uint32_t w = threadIdx.x; w < units * 4; w += blockDim.x) {
        const uint32_t u = w >> 2, k = w & 3;
        const uint32_t sb = u >> 2, g = (u >> 1) & 1, hh = u & 1;
        const uint32_t a = A[w], b = B[w], h = H[w];
        const uint32_t sc = t.s[(size_t)row * units + u];
        const float d = h2f(t.d[(size_t)row * sblocks + sb]);
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            const uint32_t c = q6_codes(a, b, h, q);
            const float ds = __fmul_rn(d, (float)(int8_t)(sc >> (8 * q)));
#pragma unroll
            for (int n = 0; n < 4; ++n) {
                const int code = (int)((c >> (8 * n)) & 0xFF) - 32;
                const uint32_t e = sb * 256 + g * 128 + q * 32 + hh * 16 + 4 * k + n;
                xs[e] = __fmul_rn(__fmul_rn(ds, (float)code), in.emb_scale);
            }
        }
    }
    (void)K;
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
__device__ void input_stage(const InputStage& in, float* xs, uint32_t K, double* red) {
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
        embed_row(in, xs, K);
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
// y = W x with W in Q4_0 and x fp32.  Each 32-element block b of x is written exactly as
//   x_j = s_b (q0_j + q1_j 2^-7 + q2_j 2^-14 + q3_j 2^-21),  s_b = 2^(ilogb(max |x_b|) - 5),
// with integer digits |q| <= 64 (every step is exact in fp32: scaling by a power of two,
// rint, and subtracting an integer within 0.5).  Then for row r and block b
//   sum_j (n_rj - 8) x_j = sum_t 2^-7t s_b sum_j n_rj q_tj  -  8 sum_j x_j,
// and the integer sums over j come from v_mfma_i32_16x16x64_i8: A = the raw nibbles n of a
// 16-row tile (lane (r, g) holds block g of row r: low nibbles feed one MFMA, high nibbles a
// second), B = the digits, with MFMA column n = (block n / 4, digit n % 4), so both MFMAs of
// a 128-column super-tile accumulate into one 16 x 16 int32 tile.  Lanes then fold the tile
// into fp32 row partials with the block scales d, reduce over the 16 columns, and the waves
// that split the super-tiles of a row tile add their partials in LDS in slice order.

typedef int v4i __attribute__((ext_vector_type(4)));
typedef unsigned v4u __attribute__((ext_vector_type(4)));
typedef unsigned v2u __attribute__((ext_vector_type(2)));

// Streaming loads of weights (read once per step): non-temporal hint.
__device__ __forceinline__ uint4 ld_stream(const uint4* p) {
    const v4u t = __builtin_nontemporal_load(reinterpret_cast<const v4u*>(p));
    return make_uint4(t.x, t.y, t.z, t.w);
}
__device__ __forceinline__ uint2 ld_stream(const uint2* p) {
    const v2u t = __builtin_nontemporal_load(reinterpret_cast<const v2u*>(p));
    return make_uint2(t.x, t.y);
}

// Digits of 8 consecutive elements v of block b (part p of 4), given the block's max |x| m:
// 8 bytes per digit t stored at dig[((st * 4 + g) * 4 + t) * 32 + 8 p].
__device__ __forceinline__ void digits8(const float (&v)[8], float m, int8_t* dig, uint32_t b, uint32_t p) {
    const int e = m > 0.0f ? ilogbf(m) : 0;
    uint32_t w[4][2] = {{0u, 0u}, {0u, 0u}, {0u, 0u}, {0u, 0u}};
#pragma unroll
    for (int k = 0; k < 8; ++k) {
        const float u = m > 0.0f ? ldexpf(v[k], 5 - e) : 0.0f;  // |u| < 64, exact
        const float q0 = rintf(u);
        float r = (u - q0) * 128.0f;
        const float q1 = rintf(r);
        r = (r - q1) * 128.0f;
        const float q2 = rintf(r);
        r = (r - q2) * 128.0f;
        const float q3 = rintf(r);
        const int sh = 8 * (k & 3);
        w[0][k >> 2] |= ((uint32_t)(int)q0 & 0xFFu) << sh;
        w[1][k >> 2] |= ((uint32_t)(int)q1 & 0xFFu) << sh;
        w[2][k >> 2] |= ((uint32_t)(int)q2 & 0xFFu) << sh;
        w[3][k >> 2] |= ((uint32_t)(int)q3 & 0xFFu) << sh;
    }
    const uint32_t st = b >> 2, g = b & 3;
#pragma unroll
    for (int t = 0; t < 4; ++t)
        *reinterpret_cast<uint2*>(dig + ((size_t)(st * 4 + g) * 4 + t) * 32 + 8 * p) = make_uint2(w[t][0], w[t][1]);
}

// Block max |x| and sum over the 4 lanes (a quad) that hold a block's 8-element parts.
__device__ __forceinline__ void quad_stats(const float (&v)[8], float& m, float& sum) {
    float mm = 0.0f, ss = 0.0f;
#pragma unroll
    for (int k = 0; k < 8; ++k) {
        mm = fmaxf(mm, fabsf(v[k]));
        ss += v[k];
    }
    mm = fmaxf(mm, __shfl_xor(mm, 1, 64));
    mm = fmaxf(mm, __shfl_xor(mm, 2, 64));
    ss += __shfl_xor(ss, 1, 64);
    ss += __shfl_xor(ss, 2, 64);
    m = mm;
    sum = ss;
}

__device__ __forceinline__ void digit_tab(DigitTab* tab, uint32_t b, float m, float sum) {
    const float s = m > 0.0f ? ldexpf(1.0f, ilogbf(m) - 5) : 0.0f;
#pragma unroll
    for (int t = 0; t < 4; ++t) tab[b * 4 + t] = DigitTab{ldexpf(s, -7 * t), t == 0 ? 8.0f * sum : 0.0f};
}

// Digits of the input vector src (K = 32 B floats, 16-byte aligned; global or LDS) for all
// nst * 4 blocks (blocks >= B are zero): four threads per block, eight elements each.
// Layout: dig[(st * 4 + g) * 4 + t][32] int8 for block b = 4 st + g, tab[b * 4 + t].
__device__ void make_digits(const float* src, uint32_t B, uint32_t nst, int8_t* dig, DigitTab* tab) {
    const uint32_t nb = nst * 4;
    for (uint32_t base = 0; base < nb * 4; base += blockDim.x) {
        const uint32_t i = base + threadIdx.x, b = i >> 2, p = i & 3;
        float v[8];
        const bool ok = b < B;
        const float4* q = reinterpret_cast<const float4*>(src + (size_t)(ok ? b : 0) * 32 + 8 * p);
        const float4 a0 = ok ? q[0] : make_float4(0.f, 0.f, 0.f, 0.f);
        const float4 a1 = ok ? q[1] : make_float4(0.f, 0.f, 0.f, 0.f);
        v[0] = a0.x; v[1] = a0.y; v[2] = a0.z; v[3] = a0.w;
        v[4] = a1.x; v[5] = a1.y; v[6] = a1.z; v[7] = a1.w;
        float m, sum;
        quad_stats(v, m, sum);  // every lane of the quad takes part, in range or not
        if (b < nb) {
            digits8(v, m, dig, b, p);
            if (p == 0) digit_tab(tab, b, m, sum);
        }
    }
}

constexpr int kQ4Ahead = 16;  // super-tiles loaded ahead per wave

struct Q4Tile {
    uint4 code;
    uint2 scale;
};

template <int T, int IN, int OUT>
__global__ __launch_bounds__(512) void q4_gemv_kernel(Q4Args a, uint32_t out_rows) {
    extern __shared__ __align__(16) uint8_t smem[];
    __shared__ double red[8];
    __shared__ float part[T][8][16];

    if (a.state && a.state[ST_STOP]) return;
    const uint32_t tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const uint32_t S = a.slices, tile = wave / S, sl = wave % S;
    const Q4View& m = (T == 2 && tile == 1) ? a.w2 : a.w;
    const uint32_t B = a.w.blocks, K = B * 32, nst = a.w.nst;
    const uint32_t per = (nst + S - 1) / S, st0 = min(nst, sl * per), st1 = min(nst, st0 + per);
    const size_t tile_base = (size_t)blockIdx.x * nst;
    const uint32_t r_ld = lane & 15, g_ld = lane >> 4;  // A operand: row, block in super-tile
    const uint32_t q = lane >> 4, n = lane & 15;         // D tile: rows 4q..4q+3, column n
    const uint32_t blk = n >> 2, t = n & 3;

    const uint4* codes = reinterpret_cast<const uint4*>(m.codes);
    const uint2* scales = reinterpret_cast<const uint2*>(m.scales);
    auto load = [&](Q4Tile (&buf)[kQ4Ahead], uint32_t c0) {
#pragma unroll
        for (int u = 0; u < kQ4Ahead; ++u) {
            const uint32_t st = c0 + u;
            if (st < st1) {
                buf[u].code = ld_stream(codes + (tile_base + st) * 64 + r_ld * 4 + g_ld);
                buf[u].scale = ld_stream(scales + (tile_base + st) * 16 + blk * 4 + q);
            }
        }
    };
    Q4Tile buf[kQ4Ahead];
    load(buf, st0);  // weights first: their latency overlaps the input stage

    const size_t xs_bytes = IN == IN_PLAIN ? 0 : (size_t)K * 4;
    int8_t* dig = reinterpret_cast<int8_t*>(smem + xs_bytes);
    DigitTab* tab = reinterpret_cast<DigitTab*>(smem + xs_bytes + (size_t)nst * 512);
    if constexpr (IN == IN_PLAIN) {
        make_digits(a.in.x, B, nst, dig, tab);
    } else {
        float* xs = reinterpret_cast<float*>(smem);
        input_stage<IN>(a.in, xs, K, red);
        make_digits(xs, B, nst, dig, tab);
    }
    __syncthreads();

    const bool bsel = (n >> 2) == q;  // B lane (k-group q, column n) is non-zero for block q only
    float acc[4] = {0.f, 0.f, 0.f, 0.f};
    const v4i zero = {0, 0, 0, 0};
    for (uint32_t c0 = st0; c0 < st1; c0 += kQ4Ahead) {
#pragma unroll
        for (int u = 0; u < kQ4Ahead; ++u) {
            const uint32_t st = c0 + u;
            if (st >= st1) break;
            const uint4 cw = buf[u].code;
            const uint2 sw = buf[u].scale;
            const v4i a1 = {(int)(cw.x & 0x0F0F0F0Fu), (int)(cw.y & 0x0F0F0F0Fu), (int)(cw.z & 0x0F0F0F0Fu),
                            (int)(cw.w & 0x0F0F0F0Fu)};
            const v4i a2 = {(int)((cw.x >> 4) & 0x0F0F0F0Fu), (int)((cw.y >> 4) & 0x0F0F0F0Fu),
                            (int)((cw.z >> 4) & 0x0F0F0F0Fu), (int)((cw.w >> 4) & 0x0F0F0F0Fu)};
            v4i b1 = zero, b2 = zero;
            if (bsel) {
                const uint4* dp = reinterpret_cast<const uint4*>(dig + ((size_t)(st * 4 + q) * 4 + t) * 32);
                const uint4 lo = dp[0], hi = dp[1];
                b1 = v4i{(int)lo.x, (int)lo.y, (int)lo.z, (int)lo.w};
                b2 = v4i{(int)hi.x, (int)hi.y, (int)hi.z, (int)hi.w};
            }
            v4i d = __builtin_amdgcn_mfma_i32_16x16x64_i8(a1, b1, zero, 0, 0, 0);
            d = __builtin_amdgcn_mfma_i32_16x16x64_i8(a2, b2, d, 0, 0, 0);
            const DigitTab tb = tab[(st * 4 + blk) * 4 + t];
            const uint16_t dh[4] = {(uint16_t)(sw.x & 0xFFFFu), (uint16_t)(sw.x >> 16), (uint16_t)(sw.y & 0xFFFFu),
                                    (uint16_t)(sw.y >> 16)};
#pragma unroll
            for (int i = 0; i < 4; ++i) acc[i] = fmaf(h2f(dh[i]), fmaf((float)d[i], tb.scale, -tb.bias), acc[i]);
        }
        if (c0 + kQ4Ahead < st1) load(buf, c0 + kQ4Ahead);
    }
    // sum the 16 columns of each row, then the slices
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int o = 8; o > 0; o >>= 1) acc[i] += __shfl_xor(acc[i], o, 16);
    if (n == 0) {
#pragma unroll
        for (int i = 0; i < 4; ++i) part[tile][sl][4 * q + i] = acc[i];
    }
    __syncthreads();
    if (tid < 16) {
        float v[T];
#pragma unroll
        for (int k = 0; k < T; ++k) {
            float s = part[k][0][tid];
            for (uint32_t j = 1; j < S; ++j) s += part[k][j][tid];
            v[k] = s;
        }
        const uint32_t row = blockIdx.x * 16 + tid;
        if (row < out_rows) {
            if constexpr (OUT == OUT_GELU) a.y[row] = gelu_mul(v[0], v[T - 1]);
            else if constexpr (OUT == OUT_ADD) a.y[row] = __fadd_rn(v[0], a.add[row]);
            else a.y[row] = v[0];
        }
    }
}

// Waves per row tile: enough waves to fill the chip (~2048), within the super-tiles and 8 per block.
static uint32_t q4_slices(uint32_t tiles, uint32_t per_tile, uint32_t nst) {
    uint32_t s = 1;
    while (s < 8 && per_tile * s * 2 <= 8 && tiles * per_tile * s < 2048 && s * 2 <= nst) s *= 2;
    return s;
}

template <int T, int IN, int OUT>
static hipError_t q4_launch2(Q4Args a, uint32_t out_rows, hipStream_t st) {
    const uint32_t tiles = (out_rows + 15) / 16;
    a.slices = q4_slices(tiles, T, a.w.nst);
    const size_t lds = (IN == IN_PLAIN ? 0 : (size_t)a.w.blocks * 32 * 4) + (size_t)a.w.nst * (512 + 128);
    hipLaunchKernelGGL((q4_gemv_kernel<T, IN, OUT>), dim3(tiles), dim3(64 * T * a.slices), lds, st, a, out_rows);
    return hipGetLastError();
}

template <int IN>
static hipError_t q4_launch1(const Q4Args& a, int out_kind, uint32_t out_rows, hipStream_t st) {
    switch (out_kind) {
        case OUT_PLAIN: return q4_launch2<1, IN, OUT_PLAIN>(a, out_rows, st);
        case OUT_GELU: return q4_launch2<2, IN, OUT_GELU>(a, out_rows, st);
        case OUT_ADD: return q4_launch2<1, IN, OUT_ADD>(a, out_rows, st);
        default: return hipErrorInvalidValue;
    }
}

hipError_t launch_q4_gemv(const Q4Args& a, int in_kind, int out_kind, uint32_t out_rows, hipStream_t s) {
    if (a.w.nst > 128) return hipErrorInvalidValue;  // columns <= 16384
    switch (in_kind) {
        case IN_PLAIN: return q4_launch1<IN_PLAIN>(a, out_kind, out_rows, s);
        case IN_NORM: return q4_launch1<IN_NORM>(a, out_kind, out_rows, s);
        case IN_RESID: return q4_launch1<IN_RESID>(a, out_kind, out_rows, s);
        case IN_EMBED: return q4_launch1<IN_EMBED>(a, out_kind, out_rows, s);
        default: return hipErrorInvalidValue;
    }
}

// ---- Q6_K head GEMV with fused greedy argmax --------------------------------------------------
//
// Lane u of every wave owns 64-weight unit u of each row (units <= 64, i.e.
// columns <= 4096), with its 64 inputs in registers.  Waves stride over rows
// R at a time; each keeps the best (value, smallest id) and a non-finite flag.
// The last block to finish reduces the per-block partials and, in step mode,
// appends the id to the session's token array and advances the position.

__device__ __forceinline__ bool better(float v, uint32_t i, float bv, uint32_t bi) {
    return v > bv || (v == bv && i < bi);
}

template <int R>
struct Q6Rows {
    uint4 a[R], b[R], h[R];
    uint32_t s[R];
    uint16_t d[R];
};

template <int R>
__device__ __forceinline__ void q6_load(Q6Rows<R>& o, const Q6View& w, uint32_t r0, uint32_t u, bool act) {
    const uint32_t sblocks = w.units / 4;
#pragma unroll
    for (int i = 0; i < R; ++i) {
        const uint32_t row = r0 + i;
        const bool ok = act && row < w.rows;
        const size_t off = ((size_t)row * w.units + u) * 16;
        o.a[i] = ok ? *reinterpret_cast<const uint4*>(w.a + off) : make_uint4(0, 0, 0, 0);
        o.b[i] = ok ? *reinterpret_cast<const uint4*>(w.b + off) : make_uint4(0, 0, 0, 0);
        o.h[i] = ok ? *reinterpret_cast<const uint4*>(w.h + off) : make_uint4(0, 0, 0, 0);
        o.s[i] = ok ? w.s[(size_t)row * w.units + u] : 0u;
        o.d[i] = ok ? w.d[(size_t)row * sblocks + (u >> 2)] : (uint16_t)0;
    }
}

template <int IN>
__global__ __launch_bounds__(256) void q6_head_kernel(HeadArgs a) {
    constexpr int R = kHeadRows;
    extern __shared__ float xs[];
    __shared__ double red[8];
    __shared__ float wv[256];
    __shared__ uint32_t wi[256], wb[256];
    __shared__ bool last;

    if (a.state && a.state[ST_STOP]) return;
    const uint32_t units = a.w.units, K = units * 64;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const bool act = (uint32_t)lane < units;
    const uint32_t u = act ? (uint32_t)lane : 0;
    const uint32_t rows = a.w.rows;
    const uint32_t stride = gridDim.x * 4 * R;
    uint32_t r0 = (blockIdx.x * 4 + wave) * R;
    Q6Rows<R> cur;
    q6_load(cur, a.w, r0, u, act);  // weights first: their latency overlaps the input stage

    if constexpr (IN == IN_PLAIN) {
        const float4* src = reinterpret_cast<const float4*>(a.in.x);
        float4* dst = reinterpret_cast<float4*>(xs);
        for (uint32_t i = threadIdx.x; i < K / 4; i += blockDim.x) dst[i] = src[i];
        __syncthreads();
    } else {
        input_stage<IN>(a.in, xs, K, red);
    }
    const uint32_t base = (u >> 2) * 256 + ((u >> 1) & 1) * 128 + (u & 1) * 16;
    float x[4][16], bias[4];
#pragma unroll
    for (int q = 0; q < 4; ++q) {
        float t = 0.0f;
#pragma unroll
        for (int j = 0; j < 16; ++j) {
            x[q][j] = act ? xs[base + q * 32 + j] : 0.0f;
            t += x[q][j];
        }
        bias[q] = 32.0f * t;
    }

    float bv = -INFINITY;
    uint32_t bi = 0xFFFFFFFFu, bad = 0;
    while (r0 < rows) {
        const uint32_t nr = r0 + stride;
        Q6Rows<R> nxt;
        q6_load(nxt, a.w, nr, u, act && nr < rows);
        float acc[R];
#pragma unroll
        for (int i = 0; i < R; ++i) {
            const uint32_t av[4] = {cur.a[i].x, cur.a[i].y, cur.a[i].z, cur.a[i].w};
            const uint32_t bw[4] = {cur.b[i].x, cur.b[i].y, cur.b[i].z, cur.b[i].w};
            const uint32_t hv[4] = {cur.h[i].x, cur.h[i].y, cur.h[i].z, cur.h[i].w};
            const float d = h2f(cur.d[i]);
            float t = 0.0f;
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                float sq = 0.0f;
#pragma unroll
                for (int k = 0; k < 4; ++k) {
                    const uint32_t c = q6_codes(av[k], bw[k], hv[k], q);
                    sq = fmaf((float)(c & 0xFFu), x[q][4 * k + 0], sq);
                    sq = fmaf((float)((c >> 8) & 0xFFu), x[q][4 * k + 1], sq);
                    sq = fmaf((float)((c >> 16) & 0xFFu), x[q][4 * k + 2], sq);
                    sq = fmaf((float)(c >> 24), x[q][4 * k + 3], sq);
                }
                const float ds = d * (float)(int8_t)(cur.s[i] >> (8 * q));
                t = fmaf(ds, sq - bias[q], t);
            }
            acc[i] = wave_sum(t);
        }
        if (lane == 0) {
#pragma unroll
            for (int i = 0; i < R; ++i) {
                const uint32_t row = r0 + i;
                if (row < rows) {
                    const float v = acc[i];
                    if (!isfinite(v)) bad = 1;
                    else if (better(v, row, bv, bi)) {
                        bv = v;
                        bi = row;
                    }
                }
            }
        }
        if (a.logits) {
            float v = acc[0];
#pragma unroll
            for (int i = 1; i < R; ++i)
                if (lane == i) v = acc[i];
            if (lane < R && r0 + lane < rows) a.logits[r0 + lane] = v;
        }
        cur = nxt;
        r0 = nr;
    }
    if (lane == 0) {
        wv[wave] = bv;
        wi[wave] = bi;
        wb[wave] = bad;
    }
    __syncthreads();
    if (threadIdx.x == 0) {
        for (int w = 1; w < 4; ++w) {
            if (better(wv[w], wi[w], bv, bi)) {
                bv = wv[w];
                bi = wi[w];
            }
            bad |= wb[w];
        }
        a.partial[blockIdx.x] = make_uint4(__float_as_uint(bv), bi, bad, 0u);
        __threadfence();
        const uint32_t ticket = atomicAdd(a.counter, 1u);
        last = ticket == gridDim.x - 1;
    }
    __syncthreads();
    if (!last) return;
    __threadfence();
    float v = -INFINITY;
    uint32_t id = 0xFFFFFFFFu, flag = 0;
    for (uint32_t b = threadIdx.x; b < gridDim.x; b += blockDim.x) {
        const uint4 p = a.partial[b];
        const float pv = __uint_as_float(p.x);
        if (better(pv, p.y, v, id)) {
            v = pv;
            id = p.y;
        }
        flag |= p.z;
    }
    wv[threadIdx.x] = v;
    wi[threadIdx.x] = id;
    wb[threadIdx.x] = flag;
    __syncthreads();
    for (uint32_t h = blockDim.x / 2; h > 0; h >>= 1) {
        if (threadIdx.x < h) {
            const uint32_t o = threadIdx.x + h;
            if (better(wv[o], wi[o], wv[threadIdx.x], wi[threadIdx.x])) {
                wv[threadIdx.x] = wv[o];
                wi[threadIdx.x] = wi[o];
            }
            wb[threadIdx.x] |= wb[o];
        }
        __syncthreads();
    }
    if (threadIdx.x == 0) {
        const uint32_t best = wi[0], flagged = wb[0] || best >= rows;
        if (a.result) {
            a.result[0] = best;
            a.result[1] = flagged;
        }
        if (a.state) {
            const uint32_t pos = a.state[ST_POS];
            uint32_t stop = flagged;
            for (uint32_t i = 0; i < a.state[ST_NSTOP]; ++i)
                if (a.stop_ids[i] == best) stop = 1u;
            a.ids[pos + 1] = best;
            if (flagged) a.state[ST_BAD] = 1u;
            if (stop) a.state[ST_STOP] = 1u;
            a.state[ST_POS] = pos + 1;
            if (a.records) {
                StepRecord r;
                r.id = best;
                r.bad = flagged;
                r.stop = stop;
                r.done = 1u;
                a.records[pos + 1] = r;
            }
        }
        *a.counter = 0u;
    }
}

// Persistent grid: at most three workgroups per CU, each wave striding over row groups.
uint32_t head_grid(uint32_t rows) {
    uint32_t per_block = 4 * kHeadRows;
    uint32_t g = (rows + per_block - 1) / per_block;
    return g > 768 ? 768 : g;
}

hipError_t launch_head(const HeadArgs& a, int in_kind, uint32_t grid, hipStream_t s) {
    const size_t lds = (size_t)a.w.units * 64 * sizeof(float);
    switch (in_kind) {
        case IN_PLAIN: hipLaunchKernelGGL(q6_head_kernel<IN_PLAIN>, dim3(grid), dim3(256), lds, s, a); break;
        case IN_NORM: hipLaunchKernelGGL(q6_head_kernel<IN_NORM>, dim3(grid), dim3(256), lds, s, a); break;
        case IN_RESID: hipLaunchKernelGGL(q6_head_kernel<IN_RESID>, dim3(grid), dim3(256), lds, s, a); break;
        default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

// ---- GQA decode attention ---------------------------------------------------------------------
//
// Grid (cmax, kv_heads), 256 threads.  Each block takes one chunk of the
// visible range [max(0, pos + 1 - window), pos] for one KV head and its GQ
// query heads.  Prologue: q-norm + NeoX RoPE of the query heads (double angle,
// double rotation, f32 result); the block whose chunk ends at pos also
// normalises and rotates the new key, optionally normalises the value, rounds
// both to fp16 and appends them at slot pos % ring.  Then scores (16 lanes per
// token), chunk softmax, and p-weighted values; chunk partials (acc, max, sum)
// are merged by the last block of the KV head.

template <int D, int GQ>
__global__ __launch_bounds__(256) void attention_kernel(AttnArgs a) {
    static_assert(D == 256, "one thread per channel");
    constexpr int NH = GQ + 2;  // query heads, then the new key and value
    __shared__ float nrm[NH][D];
    __shared__ float qs[GQ][D];
    __shared__ float scores[GQ][kAttnMaxChunkLen];
    __shared__ float vred[8][GQ][D];
    __shared__ double dred[4][NH];
    __shared__ float fred[8];
    __shared__ float cw[GQ][kAttnMaxChunks];
    __shared__ bool last;

    const uint32_t tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    if (a.state && a.state[ST_STOP]) return;
    const uint32_t pos = a.state ? a.state[ST_POS] : a.position;
    const uint32_t nvis = a.window ? min(pos + 1, a.window) : pos + 1;
    const uint32_t start = pos + 1 - nvis;
    uint32_t chunks = min(a.cmax, (nvis + a.min_chunk - 1) / a.min_chunk);
    const uint32_t clen = (nvis + chunks - 1) / chunks;
    chunks = (nvis + clen - 1) / clen;
    const uint32_t c = blockIdx.x, kvh = blockIdx.y;
    if (c >= chunks) return;
    const uint32_t t0 = start + c * clen, t1 = min(pos + 1, t0 + clen);
    const uint32_t n = t1 - t0;
    const uint32_t ring = a.ring;
    const bool append = t1 == pos + 1;  // this chunk holds the new token: append its K and V
    const int nh = append ? NH : GQ;

    // ---- prologue: RMSNorm of the query heads (and new K, V) with one block reduction, then RoPE
    float raw[NH];
#pragma unroll
    for (int h = 0; h < GQ; ++h) raw[h] = a.q_raw[(size_t)(kvh * GQ + h) * D + tid];
    raw[GQ] = append ? a.k_raw[(size_t)kvh * D + tid] : 0.0f;
    raw[GQ + 1] = append ? a.v_raw[(size_t)kvh * D + tid] : 0.0f;
    double sn = 0.0, cs = 1.0;
    if (tid < D / 2) sincos((double)pos * a.inv_freq[tid], &sn, &cs);
#pragma unroll
    for (int h = 0; h < NH; ++h) {
        const double v = wave_sum((double)raw[h] * (double)raw[h]);
        if (lane == 0) dred[wave][h] = v;
    }
    __syncthreads();
#pragma unroll
    for (int h = 0; h < NH; ++h) {
        if (h >= nh) break;
        const double ss = (dred[0][h] + dred[1][h]) + (dred[2][h] + dred[3][h]);
        if (h < GQ) nrm[h][tid] = norm_apply(raw[h], inv_rms(ss, D, a.q_eps), a.q_norm[tid]);
        else if (h == GQ) nrm[h][tid] = norm_apply(raw[h], inv_rms(ss, D, a.k_eps), a.k_norm[tid]);
        else nrm[h][tid] = a.v_norm ? (float)__dmul_rn((double)raw[h], inv_rms(ss, D, a.v_eps)) : raw[h];
    }
    __syncthreads();
    if (tid < D / 2) {
#pragma unroll
        for (int h = 0; h < GQ + 1; ++h) {
            if (h == GQ && !append) break;
            const double x = (double)nrm[h][tid], y = (double)nrm[h][tid + D / 2];
            const float r0 = (float)__dsub_rn(__dmul_rn(x, cs), __dmul_rn(y, sn));
            const float r1 = (float)__dadd_rn(__dmul_rn(x, sn), __dmul_rn(y, cs));
            if (h < GQ) {
                qs[h][tid] = r0;
                qs[h][tid + D / 2] = r1;
            } else {
                const size_t slot = ((size_t)kvh * ring + pos % ring) * D;
                a.kcache[slot + tid] = f2h(r0);
                a.kcache[slot + tid + D / 2] = f2h(r1);
            }
        }
    }
    if (append) a.vcache[((size_t)kvh * ring + pos % ring) * D + tid] = f2h(nrm[GQ + 1][tid]);
    __syncthreads();

    // ---- scores: 16 lanes per token, 16 channels per lane, two tokens in flight per group
    {
        const uint32_t grp = tid >> 4, j = tid & 15;
        float qr[GQ][16];
#pragma unroll
        for (int gi = 0; gi < GQ; ++gi)
#pragma unroll
            for (int e = 0; e < 16; ++e) qr[gi][e] = qs[gi][16 * j + e];
        for (uint32_t tb = t0 + grp; tb < t1; tb += 32) {
            uint4 k[2][2];
#pragma unroll
            for (int u = 0; u < 2; ++u) {
                const uint32_t t = tb + 16 * u;
                const uint16_t* kp = a.kcache + ((size_t)kvh * ring + (t < t1 ? t : tb) % ring) * D + 16 * j;
                k[u][0] = *reinterpret_cast<const uint4*>(kp);
                k[u][1] = *reinterpret_cast<const uint4*>(kp + 8);
            }
#pragma unroll
            for (int u = 0; u < 2; ++u) {
                const uint32_t t = tb + 16 * u;
                const uint32_t kw[8] = {k[u][0].x, k[u][0].y, k[u][0].z, k[u][0].w,
                                        k[u][1].x, k[u][1].y, k[u][1].z, k[u][1].w};
                float kf[16];
#pragma unroll
                for (int e = 0; e < 8; ++e) {
                    kf[2 * e] = h2f((uint16_t)(kw[e] & 0xFFFFu));
                    kf[2 * e + 1] = h2f((uint16_t)(kw[e] >> 16));
                }
#pragma unroll
                for (int gi = 0; gi < GQ; ++gi) {
                    float d = 0.0f;
#pragma unroll
                    for (int e = 0; e < 16; ++e) d = fmaf(qr[gi][e], kf[e], d);
#pragma unroll
                    for (int o = 8; o > 0; o >>= 1) d += __shfl_xor(d, o, 16);
                    if (j == 0 && t < t1) scores[gi][t - t0] = d * a.scale;
                }
            }
        }
    }
    __syncthreads();

    float m[GQ], l[GQ];
#pragma unroll
    for (int gi = 0; gi < GQ; ++gi) {
        float mx = -INFINITY;
        for (uint32_t i = tid; i < n; i += blockDim.x) mx = fmaxf(mx, scores[gi][i]);
        m[gi] = block_max_f(mx, fred);
        float sum = 0.0f;
        for (uint32_t i = tid; i < n; i += blockDim.x) {
            const float p = expf(scores[gi][i] - m[gi]);
            scores[gi][i] = p;
            sum += p;
        }
        l[gi] = block_sum_f(sum, fred);
    }
    __syncthreads();

    // ---- values: 32 lanes per token row, 8 channels per lane, 8 token groups, 2 rows in flight
    {
        const uint32_t tg = tid >> 5, dl = tid & 31;
        float acc[GQ][8];
#pragma unroll
        for (int gi = 0; gi < GQ; ++gi)
#pragma unroll
            for (int e = 0; e < 8; ++e) acc[gi][e] = 0.0f;
        for (uint32_t tb = t0 + tg; tb < t1; tb += 16) {
            uint4 vv[2];
#pragma unroll
            for (int u = 0; u < 2; ++u) {
                const uint32_t t = tb + 8 * u;
                vv[u] = *reinterpret_cast<const uint4*>(a.vcache + ((size_t)kvh * ring + (t < t1 ? t : tb) % ring) * D +
                                                        8 * dl);
            }
#pragma unroll
            for (int u = 0; u < 2; ++u) {
                const uint32_t t = tb + 8 * u;
                if (t >= t1) break;
                const uint32_t vw[4] = {vv[u].x, vv[u].y, vv[u].z, vv[u].w};
                float vf[8];
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    vf[2 * e] = h2f((uint16_t)(vw[e] & 0xFFFFu));
                    vf[2 * e + 1] = h2f((uint16_t)(vw[e] >> 16));
                }
#pragma unroll
                for (int gi = 0; gi < GQ; ++gi) {
                    const float p = scores[gi][t - t0];
#pragma unroll
                    for (int e = 0; e < 8; ++e) acc[gi][e] = fmaf(p, vf[e], acc[gi][e]);
                }
            }
        }
#pragma unroll
        for (int gi = 0; gi < GQ; ++gi)
#pragma unroll
            for (int e = 0; e < 8; ++e) vred[tg][gi][8 * dl + e] = acc[gi][e];
    }
    __syncthreads();
    float o[GQ];
#pragma unroll
    for (int gi = 0; gi < GQ; ++gi) {
        float t = 0.0f;
#pragma unroll
        for (int g = 0; g < 8; ++g) t += vred[g][gi][tid];
        o[gi] = t;
    }
    if (chunks == 1) {
#pragma unroll
        for (int gi = 0; gi < GQ; ++gi) a.out[(size_t)(kvh * GQ + gi) * D + tid] = o[gi] / l[gi];
        return;
    }

    // ---- split-K merge: the last block of this KV head combines the chunk partials
    const size_t stride = (size_t)GQ * (D + 2);
    float* mine = a.part + ((size_t)kvh * a.cmax + c) * stride;
#pragma unroll
    for (int gi = 0; gi < GQ; ++gi) {
        mine[gi * (D + 2) + tid] = o[gi];
        if (tid == 0) {
            mine[gi * (D + 2) + D] = m[gi];
            mine[gi * (D + 2) + D + 1] = l[gi];
        }
    }
    __syncthreads();
    if (tid == 0) {
        __threadfence();
        const uint32_t ticket = atomicAdd(a.counters + kvh, 1u);
        last = ticket == chunks - 1;
    }
    __syncthreads();
    if (!last) return;
    __threadfence();
    const float* all = a.part + (size_t)kvh * a.cmax * stride;
    // chunk maxima and sums into LDS (one load per thread), then the weights exp(m_c - M)
    for (uint32_t i = tid; i < chunks * GQ; i += blockDim.x) {
        const uint32_t k = i / GQ, gi = i % GQ;
        cw[gi][k] = all[k * stride + gi * (D + 2) + D];
        vred[0][gi][k] = all[k * stride + gi * (D + 2) + D + 1];
    }
    __syncthreads();
    float M[GQ], L[GQ];
#pragma unroll
    for (int gi = 0; gi < GQ; ++gi) {
        M[gi] = -INFINITY;
        for (uint32_t k = 0; k < chunks; ++k) M[gi] = fmaxf(M[gi], cw[gi][k]);
    }
    __syncthreads();
    for (uint32_t i = tid; i < chunks * GQ; i += blockDim.x) {
        const uint32_t k = i / GQ, gi = i % GQ;
        cw[gi][k] = expf(cw[gi][k] - M[gi]);
    }
    __syncthreads();
#pragma unroll
    for (int gi = 0; gi < GQ; ++gi) {
        L[gi] = 0.0f;
        for (uint32_t k = 0; k < chunks; ++k) L[gi] = fmaf(cw[gi][k], vred[0][gi][k], L[gi]);
        float acc = 0.0f;
#pragma unroll 8
        for (uint32_t k = 0; k < chunks; ++k) acc = fmaf(cw[gi][k], all[k * stride + gi * (D + 2) + tid], acc);
        a.out[(size_t)(kvh * GQ + gi) * D + tid] = acc / L[gi];
    }
    if (tid == 0) a.counters[kvh] = 0u;
}

hipError_t launch_attention(const AttnArgs& a, uint32_t group, uint32_t head_width, hipStream_t s) {
    if (head_width != 256) return hipErrorInvalidValue;
    const dim3 grid(a.cmax, a.kv_heads);
    switch (group) {
        case 1: hipLaunchKernelGGL((attention_kernel<256, 1>), grid, dim3(256), 0, s, a); break;
        case 2: hipLaunchKernelGGL((attention_kernel<256, 2>), grid, dim3(256), 0, s, a); break;
        case 4: hipLaunchKernelGGL((attention_kernel<256, 4>), grid, dim3(256), 0, s, a); break;
        default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

// ---- small kernels ----------------------------------------------------------------------------

// One block per vector: y = f32(x * rsqrt(mean(x^2) + eps) * w), reduction in double.
__global__ __launch_bounds__(256) void rmsnorm_kernel(const float* x, const float* w, float* y, uint32_t width,
                                                      float eps) {
    __shared__ double red[8];
    const float* xv = x + (size_t)blockIdx.x * width;
    float* yv = y + (size_t)blockIdx.x * width;
    double ss = 0.0;
    for (uint32_t i = threadIdx.x; i < width; i += blockDim.x) ss += (double)xv[i] * (double)xv[i];
    const double r = inv_rms(block_sum_d(ss, red), width, eps);
    for (uint32_t i = threadIdx.x; i < width; i += blockDim.x) yv[i] = norm_apply(xv[i], r, w[i]);
}

hipError_t launch_rmsnorm(const float* x, const float* w, float* y, uint32_t width, uint32_t vectors, float eps,
                          hipStream_t s) {
    hipLaunchKernelGGL(rmsnorm_kernel, dim3(vectors), dim3(256), 0, s, x, w, y, width, eps);
    return hipGetLastError();
}

// One block: y = (f32(rms(x) * w_a) + res) * scale (w_a null: (x + res) * scale).
__global__ __launch_bounds__(256) void resid_kernel(InputStage in, uint32_t width, float* y) {
    __shared__ double red[8];
    double ra = 1.0;
    if (in.w_a) {
        double sa = 0.0;
        for (uint32_t i = threadIdx.x; i < width; i += blockDim.x) sa += (double)in.x[i] * (double)in.x[i];
        ra = inv_rms(block_sum_d(sa, red), width, in.eps_a);
    }
    for (uint32_t i = threadIdx.x; i < width; i += blockDim.x) {
        const float t = in.w_a ? norm_apply(in.x[i], ra, in.w_a[i]) : in.x[i];
        y[i] = __fmul_rn(__fadd_rn(t, in.res[i]), in.scale);
    }
}

hipError_t launch_resid(const InputStage& in, uint32_t width, float* y, hipStream_t s) {
    hipLaunchKernelGGL(resid_kernel, dim3(1), dim3(256), 0, s, in, width, y);
    return hipGetLastError();
}

__global__ void advance_kernel(uint32_t* state) { state[ST_POS] += 1u; }

hipError_t launch_advance(uint32_t* state, hipStream_t s) {
    hipLaunchKernelGGL(advance_kernel, dim3(1), dim3(1), 0, s, state);
    return hipGetLastError();
}

}  // namespace af
