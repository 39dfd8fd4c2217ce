// Batched prefill kernels for gfx950: up to kBatchMax prompt tokens through a layer with every
// weight read once for the whole batch (crates/cuda-backend/src/batch.rs, kernels/ada/q4_batch.cu
// in the reference, which runs the same per-token arithmetic as its single-token kernels; here the
// batch runs its own arithmetic, within the reference's tolerance of the FP64 oracle).
//
// A layer's batch is a chain of launches: the digit image of every token's GEMV input
// (batch_digits_kernel, with the residual and RMSNorm prologues), the Q4_0 GEMM over all tokens
// (batch_gemm_kernel), the attention of all tokens (attention_kernel with one grid z-slice per
// token, after a pass that appends every token's K and V), and so on per phase.
//
// The GEMM runs on the int8 matrix cores as the decode step does, with the batch in the MFMA's
// M dimension: v_mfma_i32_16x16x32_i8 with A = the digit planes of four tokens (row m = 4 t + i:
// digit i of token t) over one 32-weight block (k), B = the block's 32 nibble codes of 16 weight
// rows.  Each lane then holds the four digit sums of one (token, row) pair of that block, which it
// folds with the block's input scales and weight scale.  One block per MFMA, so nothing in an MFMA
// is zero padding.
#include "device.h"

namespace af {

namespace {

constexpr uint32_t kThreads = 512;

// Table entry of a block with max |x| m and element sum `sum`.
__device__ __forceinline__ BlockTab block_tab_of(float m, float sum) {
    const float s = m > 0.0f ? ldexpf(1.0f, ilogbf(m) - 5) : 0.0f;
    return BlockTab{ldexpf(s, -14), ldexpf(s, -21), -8.0f * sum, 0.0f};
}

}  // namespace

// ---- digit images of a batch --------------------------------------------------------------------

// One workgroup per token t.  The input vector of the GEMV that follows:
//   BI_PLAIN: x_t;
//   BI_RESID: v_t = (f32(rms(x_t) w_a) + res_t) * scale (w_a null: (x_t + res_t) * scale), stored to
//             x_out_t (the residual stream), then f32(rms(v_t) w_n);
//   BI_EMBED: v_t = table row ids[pos0 + t] * emb_scale, stored to x_out_t, then f32(rms(v_t) w_n).
// RMSNorm sums of squares and products in double, f32 results (crates/domain/src/rms_norm.rs:24-41).
// The image: for block b (32 elements) of token t, digit plane i at img[((b T + t) 4 + i) 32], then
// after all planes the block's BlockTab {s 2^-14, s 2^-21, -8 sum_j x_j} at tabs[b T + t]; blocks
// past the vector (up to nb) are zero.
__global__ __launch_bounds__(512) void batch_digits_kernel(BatchIn in) {
    extern __shared__ __align__(16) float xs[];  // [K]
    __shared__ double red[8];
    const uint32_t t = blockIdx.x, tid = threadIdx.x, K = in.K, T = in.T;
    const float* x = in.x ? in.x + (size_t)t * in.stride : nullptr;
    if (in.mode == BI_EMBED) {
        embed_row_at(in.table, gp(in.ids)[in.pos0 + t], in.emb_scale, xs, tid, kThreads);
    } else {
        for (uint32_t i = tid; i < K; i += kThreads) xs[i] = x[i];
    }
    __syncthreads();
    if (in.mode == BI_RESID) {
        double ra = 1.0;
        if (in.w_a) {
            double sa = 0.0;
            for (uint32_t i = tid; i < K; i += kThreads) sa += (double)xs[i] * (double)xs[i];
            ra = inv_rms(block_sum_d(sa, red), K, in.eps_a);
        }
        const float* res = in.res + (size_t)t * in.stride;
        for (uint32_t i = tid; i < K; i += kThreads) {
            const float u = in.w_a ? norm_apply(xs[i], ra, in.w_a[i]) : xs[i];
            xs[i] = __fmul_rn(__fadd_rn(u, res[i]), in.scale);
        }
        __syncthreads();
    }
    if (in.mode != BI_PLAIN) {
        float* xo = in.x_out + (size_t)t * in.stride;
        for (uint32_t i = tid; i < K; i += kThreads) {
            xo[i] = xs[i];
            if (in.snap) in.snap[(size_t)t * in.snap_stride + i] = xs[i];
        }
    }
    double rn = 1.0;
    if (in.w_n) {
        double ss = 0.0;
        for (uint32_t i = tid; i < K; i += kThreads) ss += (double)xs[i] * (double)xs[i];
        rn = inv_rms(block_sum_d(ss, red), K, in.eps_n);
    }
    // each quad of threads holds one 32-element block (8 consecutive elements per thread)
    int8_t* planes = in.img;
    BlockTab* tabs = reinterpret_cast<BlockTab*>(in.img + (size_t)in.nb * T * 128);
    for (uint32_t o = tid; o < in.nb * 4; o += kThreads) {
        const uint32_t b = o >> 2, p = o & 3;
        float v[8];
#pragma unroll
        for (int k = 0; k < 8; ++k) {
            const uint32_t e = 8 * o + k;
            const float u = e < K ? xs[e] : 0.0f;
            v[k] = e < K && in.w_n ? norm_apply(u, rn, in.w_n[e]) : u;
        }
        float m, sum;
        quad_stats(v, m, sum);
        uint32_t w[4][2];
        digit_words(v, m, w);
#pragma unroll
        for (int i = 0; i < 4; ++i)
            *reinterpret_cast<v2u*>(planes + (((size_t)b * T + t) * 4 + i) * 32 + 8 * p) = v2u{w[i][0], w[i][1]};
        if (p == 0) tabs[(size_t)b * T + t] = block_tab_of(m, sum);
    }
}

// ---- Q4_0 GEMM over a batch ---------------------------------------------------------------------

// One workgroup per 16-row tile (for a gate/up pair, the same tile of both matrices); its eight
// waves split the tile's super-tiles.  Lane l holds, per group of four tokens, the partial dot
// product of token 4 g + l / 16 with row l % 16.  P: matrices (1, or 2 for gate/up); G: token groups.
template <int P, int G>
__global__ __launch_bounds__(512) void batch_gemm_kernel(BatchGemm a) {
    __shared__ float red[8][P][4 * G][16];
    const uint32_t tid = threadIdx.x, lane = tid & 63, wave = wave_id();
    const uint32_t rt = blockIdx.x, nst = a.w.nst, T = a.T;
    const uint32_t per = (nst + 7) / 8, st0 = min(nst, wave * per), st1 = min(nst, st0 + per);
    const uint32_t row = lane & 15, kq = lane >> 4;        // B operand: column row, k-range 8 kq
    const uint32_t ta = (lane & 15) >> 2, ia = lane & 3;   // A operand: token 4 g + ta, digit ia
    const uint32_t tl = lane >> 4;                         // D: token 4 g + tl of row `row`
    const int8_t* planes = a.img;
    const BlockTab* tabs = reinterpret_cast<const BlockTab*>(a.img + (size_t)nst * 4 * T * 128);
    float acc[P][G];
#pragma unroll
    for (int q = 0; q < P; ++q)
#pragma unroll
        for (int g = 0; g < G; ++g) acc[q][g] = 0.0f;
    for (uint32_t st = st0; st < st1; ++st) {
#pragma unroll
        for (uint32_t blk = 0; blk < 4; ++blk) {
            const uint32_t b = st * 4 + blk;
            long B[P];
            float d[P];
#pragma unroll
            for (int q = 0; q < P; ++q) {
                const Q4View& m = q ? a.w2 : a.w;
                const size_t rec = ((size_t)rt * nst + st) * 4 + blk;
                const v2u c = *gp(reinterpret_cast<const v2u*>(m.codes + rec * 256 + row * 16 + 8 * (kq & 1)));
                const uint32_t sh = kq >= 2 ? 4u : 0u;
                const uint32_t lo = (c.x >> sh) & 0x0F0F0F0Fu, hi = (c.y >> sh) & 0x0F0F0F0Fu;
                B[q] = (long)(((uint64_t)hi << 32) | lo);
                d[q] = h2f(gp(m.scales)[rec * 16 + row]);
            }
#pragma unroll
            for (int g = 0; g < G; ++g) {
                const uint32_t tA = 4 * g + ta, tD = 4 * g + tl;
                long A = 0;
                if (tA < T) {
                    const v2u v = *gp(reinterpret_cast<const v2u*>(planes + (((size_t)b * T + tA) * 4 + ia) * 32 + 8 * kq));
                    A = (long)(((uint64_t)v.y << 32) | v.x);
                }
                const BlockTab tb = tD < T ? tabs[(size_t)b * T + tD] : BlockTab{0.0f, 0.0f, 0.0f, 0.0f};
                const v4i zero4 = {0, 0, 0, 0};
#pragma unroll
                for (int q = 0; q < P; ++q) {
                    const v4i D = __builtin_amdgcn_mfma_i32_16x16x32_i8(A, B[q], zero4, 0, 0, 0);
                    // 2^14 D0 + 2^7 D1 + D2 is exact in int32 (|D_i| <= 32 * 15 * 64)
                    const int I = (D[0] << 14) + (D[1] << 7) + D[2];
                    float in = fmaf((float)I, tb.s14, tb.nbias);
                    in = fmaf((float)D[3], tb.s21, in);
                    acc[q][g] = fmaf(d[q], in, acc[q][g]);
                }
            }
        }
    }
#pragma unroll
    for (int q = 0; q < P; ++q)
#pragma unroll
        for (int g = 0; g < G; ++g) red[wave][q][4 * g + tl][row] = acc[q][g];
    __syncthreads();
    // one thread per (token, row): the waves' partials in wave order, then the epilogue
    for (uint32_t i = tid; i < T * 16; i += kThreads) {
        const uint32_t t = i >> 4, r = i & 15, y_row = rt * 16 + r;
        float v[P];
#pragma unroll
        for (int q = 0; q < P; ++q) {
            float s = red[0][q][t][r];
#pragma unroll
            for (int w = 1; w < 8; ++w) s += red[w][q][t][r];
            v[q] = s;
        }
        if (y_row >= a.rows) continue;
        float* y = a.y + (size_t)t * a.y_stride + y_row;
        if constexpr (P == 2) *y = gelu_mul(v[0], v[1]);
        else if (a.add) *y = __fadd_rn(v[0], a.add[(size_t)t * a.y_stride + y_row]);
        else *y = v[0];
    }
}

// ---- launchers ----------------------------------------------------------------------------------

size_t batch_image_bytes(uint32_t nst, uint32_t tokens) { return (size_t)nst * 4 * tokens * (128 + 16); }

hipError_t launch_batch_digits(const BatchIn& in, hipStream_t s) {
    if (in.T == 0 || in.T > kBatchMax || in.K > 16384 || in.nb * 32 < in.K) return hipErrorInvalidValue;
    hipLaunchKernelGGL(batch_digits_kernel, dim3(in.T), dim3(kThreads), (size_t)in.K * 4, s, in);
    return hipGetLastError();
}

template <int P>
static hipError_t gemm_launch(const BatchGemm& a, hipStream_t s) {
    const dim3 grid((a.rows + 15) / 16);
    switch ((a.T + 3) / 4) {
        case 1: hipLaunchKernelGGL((batch_gemm_kernel<P, 1>), grid, dim3(kThreads), 0, s, a); break;
        case 2: hipLaunchKernelGGL((batch_gemm_kernel<P, 2>), grid, dim3(kThreads), 0, s, a); break;
        case 3:
        case 4: hipLaunchKernelGGL((batch_gemm_kernel<P, 4>), grid, dim3(kThreads), 0, s, a); break;
        case 5:
        case 6:
        case 7:
        case 8: hipLaunchKernelGGL((batch_gemm_kernel<P, 8>), grid, dim3(kThreads), 0, s, a); break;
        default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

hipError_t launch_batch_gemm(const BatchGemm& a, bool gelu_pair, hipStream_t s) {
    if (a.T == 0 || a.T > kBatchMax || a.rows == 0) return hipErrorInvalidValue;
    return gelu_pair ? gemm_launch<2>(a, s) : gemm_launch<1>(a, s);
}

}  // namespace af
