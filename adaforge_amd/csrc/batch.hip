// Batched prefill kernels for gfx950: up to kBatchMax prompt tokens through a layer with every
// weight read once for the whole batch (crates/cuda-backend/src/batch.rs, kernels/ada/q4_batch.cu
// in the reference).  A layer's batch is a chain of launches: the input image of every token's GEMV
// input (batch_input_kernel, with the residual and RMSNorm prologues), the Q4_0 GEMM over all tokens
// (batch_gemm_kernel, then batch_reduce_kernel when the GEMM splits K across workgroups), and the
// attention of all tokens (attention_kernel with one grid z-slice per token, after a pass that
// appends every token's K and V).
//
// Each token's GEMM input is written as two fp16 halves per 32-element block: with u the block
// scaled by 2^(14 - e) (e = ilogb of the block's max |x|, so that |u| < 2^15), hi = fp16(u) and
// lo = fp16(u - hi), both rounded to nearest even; hi + lo holds u to about 2^-23 of the block's max.  The GEMM runs on the
// fp16 matrix cores with the tokens in the MFMA's M dimension: v_mfma_f32_16x16x32_f16 with A = the
// hi (then the lo) halves of 16 tokens over one 32-weight block (k) and B = the block's weights
// n - 8 of 16 rows as fp16 (exact: each nibble placed in the mantissa of 1024 + n, then 1032
// subtracted), both MFMAs accumulating into one fp32 tile, so D[t][r] = sum_j u_j(t) (n_rj - 8) with
// every product exact.  Each lane adds d_r 2^(e - 14) D[t][r] to its fp32 partial per block.
#include "device.h"

namespace af {

typedef _Float16 v8h __attribute__((ext_vector_type(8)));
typedef _Float16 v2h __attribute__((ext_vector_type(2)));

namespace {

constexpr uint32_t kGemmThreads = 256;  // four waves splitting the blocks of the workgroup's K range
constexpr uint32_t kGemmTargetGrid = 512;

uint32_t padded_tokens(uint32_t T) { return (T + 15) / 16 * 16; }

// Work split of a GEMM: R row tiles per workgroup, S workgroups along K (partials summed by
// batch_reduce_kernel), so that about kGemmTargetGrid workgroups share the weight stream and each
// wave keeps at least two blocks.
struct GemmPlan {
    uint32_t R, S;
};
// The input image is read by every workgroup of a K range, R row tiles at a time, so R sets its
// reuse: up to 8 tiles (4 of each matrix of a gate/up pair) while at least 32 row groups remain.
GemmPlan gemm_plan(uint32_t rows, uint32_t blocks, bool pair) {
    const uint32_t tiles = (rows + 15) / 16, r_max = pair ? 4 : 8;
    uint32_t R = 1;
    while (R < r_max && tiles >= 64 * R) R *= 2;
    const uint32_t wgs = (tiles + R - 1) / R;
    uint32_t S = std::max<uint32_t>(1, std::min<uint32_t>(32, (kGemmTargetGrid + wgs - 1) / wgs));
    S = std::max<uint32_t>(1, std::min(S, blocks / 8));
    return GemmPlan{R, S};
}

}  // namespace

// ---- input images of a batch --------------------------------------------------------------------
//
// Image of K = 32 nb inputs for Tp tokens: hi [nb][Tp][32] fp16, then lo [nb][Tp][32] fp16, then
// [nb][Tp] floats 2^(e - 14) (0 for an all-zero block and for padding tokens).  A quad of threads
// (8 elements each) writes one block.

// The halves and the scale of block b of token t from the 8 elements v of part p (all four lanes of
// the quad take part).
__device__ __forceinline__ void block_halves(const float (&v)[8], uint32_t b, uint32_t p, uint32_t t, uint32_t Tp,
                                             _Float16* hi, _Float16* lo, float* inv) {
    float m, sum;
    quad_stats(v, m, sum);
    const int e = m > 0.0f ? ilogbf(m) : 0;
    uint32_t hw[4], lw[4];
#pragma unroll
    for (int k = 0; k < 4; ++k) {
        const float u0 = ldexpf(v[2 * k], 14 - e), u1 = ldexpf(v[2 * k + 1], 14 - e);
        const _Float16 h0 = (_Float16)u0, h1 = (_Float16)u1;
        const _Float16 l0 = (_Float16)(u0 - (float)h0), l1 = (_Float16)(u1 - (float)h1);
        hw[k] = (uint32_t)__builtin_bit_cast(uint16_t, h0) | (uint32_t)__builtin_bit_cast(uint16_t, h1) << 16;
        lw[k] = (uint32_t)__builtin_bit_cast(uint16_t, l0) | (uint32_t)__builtin_bit_cast(uint16_t, l1) << 16;
    }
    const size_t at = ((size_t)b * Tp + t) * 32 + 8 * p;
    *reinterpret_cast<v4u*>(hi + at) = v4u{hw[0], hw[1], hw[2], hw[3]};
    *reinterpret_cast<v4u*>(lo + at) = v4u{lw[0], lw[1], lw[2], lw[3]};
    if (p == 0) inv[(size_t)b * Tp + t] = m > 0.0f ? ldexpf(1.0f, e - 14) : 0.0f;
}

// One workgroup per token t < Tp (tokens T..Tp-1 write zeros).  The input vector of the GEMV that
// follows:
//   BI_PLAIN: x_t (f32(rms(x_t) w_n) with w_n);
//   BI_RESID: v_t = (f32(rms(x_t) w_a) + res_t) * scale (w_a null: (x_t + res_t) * scale), stored to
//             x_out_t (the residual stream), then f32(rms(v_t) w_n);
//   BI_EMBED: v_t = table row ids[pos0 + t] * emb_scale, stored to x_out_t, then f32(rms(v_t) w_n).
// RMSNorm sums of squares and products in double, f32 results (crates/domain/src/rms_norm.rs:24-41).
// Thread j holds octets j, j + 512, ... (NO of them) in registers, and every global load of the
// token (x, res and both norm weights) is issued before the first reduction, so the kernel waits
// for memory once.
// PS: x comes from in.parts split-K partial planes (NO == 1 only).
template <int NO, bool PS>
__global__ __launch_bounds__(512) void batch_input_kernel(BatchIn in) {
    extern __shared__ __align__(16) float xs[];  // [K], BI_EMBED only
    __shared__ double red[8];
    const uint32_t t = blockIdx.x, tid = threadIdx.x, K = in.K, nb = K / 32, no = K / 8, Tp = gridDim.x;
    _Float16* hi = reinterpret_cast<_Float16*>(in.img);
    _Float16* lo = hi + (size_t)nb * Tp * 32;
    float* inv = reinterpret_cast<float*>(lo + (size_t)nb * Tp * 32);
    if (t >= in.T) {
        for (uint32_t o = tid; o < nb * 4; o += blockDim.x) {
            const uint32_t b = o >> 2, p = o & 3;
            const size_t at = ((size_t)b * Tp + t) * 32 + 8 * p;
            *reinterpret_cast<v4u*>(hi + at) = v4u{0u, 0u, 0u, 0u};
            *reinterpret_cast<v4u*>(lo + at) = v4u{0u, 0u, 0u, 0u};
            if (p == 0) inv[(size_t)b * Tp + t] = 0.0f;
        }
        return;
    }
    const bool resid = in.mode == BI_RESID, embed = in.mode == BI_EMBED;
    const float4 z4 = make_float4(0.f, 0.f, 0.f, 0.f);
    float4 x[NO][2], r[NO][2], wa[NO][2], wn[NO][2];
#pragma unroll
    for (int j = 0; j < NO; ++j) {
        const uint32_t o = tid + 512 * j;
        x[j][0] = x[j][1] = r[j][0] = r[j][1] = wa[j][0] = wa[j][1] = wn[j][0] = wn[j][1] = z4;
        if (o < no) {
            if constexpr (PS) {
                // every plane's loads issued first, then the sums in split order
                const float* p0 = in.part + (size_t)t * in.part_row + 8 * o;
                const size_t plane = (size_t)gridDim.x * in.part_row;
                float4 pv[kDeferParts][2];
#pragma unroll
                for (int k = 0; k < (int)kDeferParts; ++k) {
                    if ((uint32_t)k < in.parts) {
                        pv[k][0] = reinterpret_cast<const float4*>(p0 + k * plane)[0];
                        pv[k][1] = reinterpret_cast<const float4*>(p0 + k * plane)[1];
                    }
                }
                x[j][0] = pv[0][0];
                x[j][1] = pv[0][1];
#pragma unroll
                for (int k = 1; k < (int)kDeferParts; ++k) {
                    if ((uint32_t)k < in.parts) {
#pragma unroll
                        for (int h = 0; h < 2; ++h) {
                            x[j][h].x += pv[k][h].x;
                            x[j][h].y += pv[k][h].y;
                            x[j][h].z += pv[k][h].z;
                            x[j][h].w += pv[k][h].w;
                        }
                    }
                }
            } else if (!embed) {
                const float4* p = reinterpret_cast<const float4*>(in.x + (size_t)t * in.stride) + 2 * o;
                x[j][0] = p[0];
                x[j][1] = p[1];
            }
            if (resid) {
                const float4* p = reinterpret_cast<const float4*>(in.res + (size_t)t * in.stride) + 2 * o;
                r[j][0] = p[0];
                r[j][1] = p[1];
                if (in.w_a) {
                    wa[j][0] = reinterpret_cast<const float4*>(in.w_a)[2 * o];
                    wa[j][1] = reinterpret_cast<const float4*>(in.w_a)[2 * o + 1];
                }
            }
            if (in.w_n) {
                wn[j][0] = reinterpret_cast<const float4*>(in.w_n)[2 * o];
                wn[j][1] = reinterpret_cast<const float4*>(in.w_n)[2 * o + 1];
            }
        }
    }
    if (embed) {
        embed_row_at(in.table, gp(in.ids)[in.pos0 + t], in.emb_scale, xs, tid, blockDim.x);
        __syncthreads();
#pragma unroll
        for (int j = 0; j < NO; ++j) {
            const uint32_t o = tid + 512 * j;
            if (o < no) {
                x[j][0] = reinterpret_cast<const float4*>(xs)[2 * o];
                x[j][1] = reinterpret_cast<const float4*>(xs)[2 * o + 1];
            }
        }
    }
    if (resid) {
        double ra = 1.0;
        if (in.w_a) {
            double sa = 0.0;
#pragma unroll
            for (int j = 0; j < NO; ++j) sa += sq4(x[j][0]) + sq4(x[j][1]);
            ra = inv_rms(block_sum_d(sa, red), K, in.eps_a);
        }
#pragma unroll
        for (int j = 0; j < NO; ++j)
#pragma unroll
            for (int h = 0; h < 2; ++h)
                x[j][h] = resid4(in.w_a ? norm4(x[j][h], ra, wa[j][h]) : x[j][h], r[j][h], in.scale);
    }
    if (in.mode != BI_PLAIN) {
#pragma unroll
        for (int j = 0; j < NO; ++j) {
            const uint32_t o = tid + 512 * j;
            if (o >= no) continue;
            float4* xo = reinterpret_cast<float4*>(in.x_out + (size_t)t * in.stride) + 2 * o;
            xo[0] = x[j][0];
            xo[1] = x[j][1];
            if (in.snap) {
                float* sp = in.snap + (size_t)t * in.snap_stride + 8 * o;
                const float* v = reinterpret_cast<const float*>(&x[j][0]);
#pragma unroll
                for (int k = 0; k < 8; ++k) sp[k] = v[k];
            }
        }
    }
    double rn = 1.0;
    if (in.w_n) {
        double ss = 0.0;
#pragma unroll
        for (int j = 0; j < NO; ++j) ss += sq4(x[j][0]) + sq4(x[j][1]);
        rn = inv_rms(block_sum_d(ss, red), K, in.eps_n);
    }
    // a quad of threads holds one 32-element block (no is a multiple of 4: whole quads take part)
#pragma unroll
    for (int j = 0; j < NO; ++j) {
        const uint32_t o = tid + 512 * j;
        if (o >= no) continue;
        float v[8];
#pragma unroll
        for (int h = 0; h < 2; ++h) {
            const float4 u = in.w_n ? norm4(x[j][h], rn, wn[j][h]) : x[j][h];
            v[4 * h] = u.x;
            v[4 * h + 1] = u.y;
            v[4 * h + 2] = u.z;
            v[4 * h + 3] = u.w;
        }
        block_halves(v, o >> 2, o & 3, t, Tp, hi, lo, inv);
    }
}

// BI_PLAIN inputs without a norm: one thread per 8-element octet, grid (Tp, octets / 256).  PS: the
// input is gelu(gate) * up from a gate/up pair's deferred split-K partials.
template <bool PS>
__global__ __launch_bounds__(256) void batch_plain_input_kernel(BatchIn in) {
    const uint32_t t = blockIdx.x, o = blockIdx.y * 256 + threadIdx.x, nb = in.K / 32, Tp = gridDim.x;
    if (o >= nb * 4) return;  // whole quads: nb * 4 is a multiple of 4
    _Float16* hi = reinterpret_cast<_Float16*>(in.img);
    _Float16* lo = hi + (size_t)nb * Tp * 32;
    float* inv = reinterpret_cast<float*>(lo + (size_t)nb * Tp * 32);
    float v[8];
    if (PS && t < in.T) {
        // every plane's loads first, then each matrix's sums in split order, then gelu(gate) * up
        const float* p0 = in.part + (size_t)t * in.part_row + 8 * o;
        const size_t plane = (size_t)Tp * in.part_row;
        float4 pv[kDeferPairParts][2][2];
#pragma unroll
        for (int k = 0; k < (int)kDeferPairParts; ++k)
            if ((uint32_t)k < in.parts)
#pragma unroll
                for (int q = 0; q < 2; ++q)
#pragma unroll
                    for (int h = 0; h < 2; ++h) pv[k][q][h] = reinterpret_cast<const float4*>(p0 + (2 * k + q) * plane)[h];
        float s[2][8];
#pragma unroll
        for (int q = 0; q < 2; ++q)
#pragma unroll
            for (int h = 0; h < 2; ++h) {
                s[q][4 * h] = pv[0][q][h].x;
                s[q][4 * h + 1] = pv[0][q][h].y;
                s[q][4 * h + 2] = pv[0][q][h].z;
                s[q][4 * h + 3] = pv[0][q][h].w;
            }
#pragma unroll
        for (int k = 1; k < (int)kDeferPairParts; ++k)
            if ((uint32_t)k < in.parts)
#pragma unroll
                for (int q = 0; q < 2; ++q)
#pragma unroll
                    for (int h = 0; h < 2; ++h) {
                        s[q][4 * h] += pv[k][q][h].x;
                        s[q][4 * h + 1] += pv[k][q][h].y;
                        s[q][4 * h + 2] += pv[k][q][h].z;
                        s[q][4 * h + 3] += pv[k][q][h].w;
                    }
#pragma unroll
        for (int i = 0; i < 8; ++i) v[i] = gelu_mul(s[0][i], s[1][i]);
    } else if (t < in.T) {
        const float4* x = reinterpret_cast<const float4*>(in.x + (size_t)t * in.stride) + 2 * o;
        const float4 u0 = x[0], u1 = x[1];
        v[0] = u0.x; v[1] = u0.y; v[2] = u0.z; v[3] = u0.w;
        v[4] = u1.x; v[5] = u1.y; v[6] = u1.z; v[7] = u1.w;
    } else {
#pragma unroll
        for (int k = 0; k < 8; ++k) v[k] = 0.0f;
    }
    block_halves(v, o >> 2, o & 3, t, Tp, hi, lo, inv);
}

// ---- Q4_0 GEMM over a batch ---------------------------------------------------------------------

namespace {

// A block's input operands for a wave: the hi and lo halves of its G token groups (lane l: token
// 16 g + l % 16, elements 8 (l / 16) .. + 7) and the block scales of tokens 16 g + 4 (l / 16) + e
// (the lane's outputs).  They come from L2 (the image is shared by all
// workgroups) and are loaded one block ahead.
template <int G>
struct InOps {
    v4u hi[G], lo[G];
    v4f sc[G];  // the block scales 2^(e - 14) of the four tokens whose outputs the lane folds
};

// A block's weights for R row tiles of P matrices (lane l: row l % 16, bytes 8 ((l / 16) & 1) .. + 7 of
// the block's 16 code bytes, and the row's fp16 scale).  They stream from HBM and are loaded
// kCodeAhead blocks ahead.
template <int P, int R>
struct WOps {
    uint2 code[R][P];
    uint16_t d[R][P];
};

// weight blocks in flight per wave: 8, or 2 when a block spans 4 or more tiles
template <int P, int R>
constexpr int code_ahead() { return R * P >= 4 ? 2 : 8; }

template <int G>
__device__ __forceinline__ void load_in(InOps<G>& o, const BatchGemm& a, uint32_t b, uint32_t lane) {
    constexpr uint32_t Tp = 16 * G;
    const uint32_t m = lane & 15, kq = lane >> 4;
    const _Float16* hi = reinterpret_cast<const _Float16*>(a.img);
    const _Float16* lo = hi + (size_t)a.w.blocks * Tp * 32;
    const float* inv = reinterpret_cast<const float*>(lo + (size_t)a.w.blocks * Tp * 32);
#pragma unroll
    for (int g = 0; g < G; ++g) {
        const size_t at = ((size_t)b * Tp + 16 * g + m) * 32 + 8 * kq;
        o.hi[g] = *gp(reinterpret_cast<const v4u*>(hi + at));
        o.lo[g] = *gp(reinterpret_cast<const v4u*>(lo + at));
        o.sc[g] = *gp(reinterpret_cast<const v4f*>(inv + (size_t)b * Tp + 16 * g + 4 * kq));
    }
}

template <int P, int R>
__device__ __forceinline__ void load_w(WOps<P, R>& o, const BatchGemm& a, uint32_t b, uint32_t rt0, uint32_t last_tile,
                                       uint32_t lane) {
    const uint32_t m = lane & 15, kq = lane >> 4;
    const uint32_t per_tile = a.w.nst * 4;  // block records per row tile (tiled layout, Q4View)
#pragma unroll
    for (int r = 0; r < R; ++r) {
        const size_t rec = (size_t)min(rt0 + r, last_tile) * per_tile + b;
#pragma unroll
        for (int q = 0; q < P; ++q) {
            const Q4View& w = q ? a.w2 : a.w;
            o.code[r][q] = ld_stream(reinterpret_cast<const uint2*>(w.codes + rec * 256 + m * 16 + 8 * (kq & 1)));
            o.d[r][q] = gp(w.scales)[rec * 16 + m];
        }
    }
}

// Four nibbles (one per byte of c) as fp16 (n - 8), in two pairs: n into the mantissa of 1024 + n
// (0x6400 | n), then 1032 subtracted, exactly.
__device__ __forceinline__ void nibbles_f16(uint32_t c, v2h& p0, v2h& p1) {
    const v2h bias = {(_Float16)1032.0f, (_Float16)1032.0f};
    p0 = __builtin_bit_cast(v2h, __builtin_amdgcn_perm(0u, c, 0x0c010c00u) | 0x64006400u) - bias;
    p1 = __builtin_bit_cast(v2h, __builtin_amdgcn_perm(0u, c, 0x0c030c02u) | 0x64006400u) - bias;
}

template <int P, int G, int R>
__device__ __forceinline__ void mfma_block(const InOps<G>& x, const WOps<P, R>& w, uint32_t kq,
                                           float (&acc)[R][P][G][4]) {
    const uint32_t sh = kq >= 2 ? 4u : 0u;  // k 0..15: low nibbles, 16..31: high nibbles
    const v4f zero = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
    for (int r = 0; r < R; ++r)
#pragma unroll
        for (int q = 0; q < P; ++q) {
            v2h f0, f1, f2, f3;
            nibbles_f16((w.code[r][q].x >> sh) & 0x0F0F0F0Fu, f0, f1);
            nibbles_f16((w.code[r][q].y >> sh) & 0x0F0F0F0Fu, f2, f3);
            const v8h B = {f0.x, f0.y, f1.x, f1.y, f2.x, f2.y, f3.x, f3.y};
            const float d = h2f(w.d[r][q]);
#pragma unroll
            for (int g = 0; g < G; ++g) {
                v4f D = __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(v8h, x.hi[g]), B, zero, 0, 0, 0);
                D = __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(v8h, x.lo[g]), B, D, 0, 0, 0);
#pragma unroll
                for (int e = 0; e < 4; ++e) acc[r][q][g][e] = fmaf(d * x.sc[g][e], D[e], acc[r][q][g][e]);
            }
        }
}

template <int P>
__device__ __forceinline__ void gemm_epilogue(const BatchGemm& a, uint32_t t, uint32_t row, const float (&v)[P]) {
    float* y = a.y + (size_t)t * a.y_stride + row;
    if constexpr (P == 2) *y = gelu_mul(v[0], v[1]);
    else if (a.add) *y = __fadd_rn(v[0], a.add[(size_t)t * a.y_stride + row]);
    else *y = v[0];
}

}  // namespace

// Grid (ceil(tiles / R), S): workgroup (x, s) takes row tiles R x .. R x + R - 1 (for a gate/up pair,
// those tiles of both matrices) over K range s of S; its four waves split the range's blocks and add
// their partials in LDS in wave order.  Each wave streams its blocks through a two-stage register
// pipeline (the next block's loads in flight while the current block's MFMAs run).  With S = 1 the
// workgroup writes y; otherwise it writes its partials for batch_reduce_kernel.
template <int P, int G, int R>
__global__ __launch_bounds__(256) void batch_gemm_kernel(BatchGemm a) {
    constexpr uint32_t Tp = 16 * G;
    __shared__ float red[4][R][P][Tp][16];
    const uint32_t tid = threadIdx.x, lane = tid & 63, wave = wave_id(), kq = lane >> 4;
    const uint32_t tiles = (a.w.rows + 15) / 16, rt0 = blockIdx.x * R, S = gridDim.y, split = blockIdx.y;
    const uint32_t nb = a.w.blocks;
    const uint32_t s0 = nb * split / S, s1 = nb * (split + 1) / S;
    const uint32_t b0 = s0 + (s1 - s0) * wave / 4, b1 = s0 + (s1 - s0) * (wave + 1) / 4;
    float acc[R][P][G][4];
#pragma unroll
    for (int r = 0; r < R; ++r)
#pragma unroll
        for (int q = 0; q < P; ++q)
#pragma unroll
            for (int g = 0; g < G; ++g)
#pragma unroll
                for (int e = 0; e < 4; ++e) acc[r][q][g][e] = 0.0f;
    // weights kCodeAhead blocks ahead in a register ring, inputs one block ahead (ping-pong)
    constexpr int kCodeAhead = code_ahead<P, R>();
    WOps<P, R> wr[kCodeAhead];
    InOps<G> xi[2];
    const uint32_t last_b = nb - 1;
#pragma unroll
    for (int u = 0; u < kCodeAhead; ++u) load_w(wr[u], a, min(b0 + u, last_b), rt0, tiles - 1, lane);
    if (b0 < b1) load_in(xi[0], a, b0, lane);
    for (uint32_t b = b0; b < b1; b += kCodeAhead) {
#pragma unroll
        for (int u = 0; u < kCodeAhead; ++u) {
            const uint32_t bb = b + u;
            if (bb >= b1) break;
            if (bb + 1 < b1) load_in(xi[(u + 1) & 1], a, bb + 1, lane);
            mfma_block(xi[u & 1], wr[u], kq, acc);
            load_w(wr[u], a, min(bb + kCodeAhead, last_b), rt0, tiles - 1, lane);
        }
    }
#pragma unroll
    for (int r = 0; r < R; ++r)
#pragma unroll
        for (int q = 0; q < P; ++q)
#pragma unroll
            for (int g = 0; g < G; ++g)
#pragma unroll
                for (int e = 0; e < 4; ++e) red[wave][r][q][16 * g + 4 * kq + e][lane & 15] = acc[r][q][g][e];
    __syncthreads();
    const size_t prow = (size_t)tiles * 16;
    for (uint32_t i = tid; i < R * Tp * 16; i += kGemmThreads) {
        const uint32_t r = i / (Tp * 16), t = (i / 16) % Tp, n = i & 15;
        const uint32_t tile = rt0 + r, row = tile * 16 + n;
        if (tile >= tiles || t >= a.T) continue;
        float v[P];
#pragma unroll
        for (int q = 0; q < P; ++q) v[q] = ((red[0][r][q][t][n] + red[1][r][q][t][n]) + red[2][r][q][t][n]) + red[3][r][q][t][n];
        if (S > 1) {
#pragma unroll
            for (int q = 0; q < P; ++q) a.part[((size_t)(split * P + q) * Tp + t) * prow + row] = v[q];
        } else if (row < a.w.rows) {
            gemm_epilogue<P>(a, t, row, v);
        }
    }
}

// y from the S split-K partials of batch_gemm_kernel, summed in split order; one thread per (t, row).
template <int P>
__global__ __launch_bounds__(256) void batch_reduce_kernel(BatchGemm a, uint32_t S, uint32_t Tp) {
    const uint32_t rows = a.w.rows, i = blockIdx.x * 256 + threadIdx.x;
    if (i >= a.T * rows) return;
    const uint32_t t = i / rows, row = i % rows;
    const size_t prow = (size_t)(rows + 15) / 16 * 16;
    float v[P];
#pragma unroll
    for (int q = 0; q < P; ++q) {
        float s = a.part[((size_t)q * Tp + t) * prow + row];
        for (uint32_t k = 1; k < S; ++k) s += a.part[((size_t)(k * P + q) * Tp + t) * prow + row];
        v[q] = s;
    }
    gemm_epilogue<P>(a, t, row, v);
}

// ---- attention of a batch ----------------------------------------------------------------------
//
// Grid (nchunks, kv_heads, query tiles): workgroup (c, h, j) takes query tile j of KV head h (queries
// i = t group + g of its tokens t and query heads h group + g, 16 per tile) against chunk c of the
// keys, streamed in sub-chunks of KC keys through LDS, with an online softmax.  Both products run
// on the fp16 matrix cores (v_mfma_f32_16x16x32_f16, fp32 accumulation): the cached K and V are
// fp16 already, and the fp32 queries and probabilities enter as fp16 pairs hi + lo (hi = f16(x),
// lo = f16(x - hi)) after scaling by a power of two (queries to below 32 in magnitude, probabilities
// by 2^14), so each operand keeps about 22 significant bits and every product is exact in fp32.

namespace {


__device__ __forceinline__ void split_f16(float x, _Float16& hi, _Float16& lo) {
    hi = (_Float16)x;
    lo = (_Float16)(x - (float)hi);  // exact in fp32: hi is the nearest fp16 to x
}

}  // namespace

template <int D, int KC>
__global__ __launch_bounds__(256) void batch_attention_kernel(BatchAttn a) {
    constexpr int KP = D + 8;         // row stride of K and of the query planes (halves)
    constexpr int VP = KC + 8;        // row stride of V^T and of the probability planes (halves)
    constexpr int KT = KC / 16;       // 16-key score tiles
    constexpr int DH = 4 / KT;        // head-width parts per score tile (four waves)
    constexpr int DS = D / 32 / DH;   // MFMA steps per part
    constexpr int NT = D / 64;        // 16-channel output tiles per wave
    __shared__ __align__(16) _Float16 qh[16 * KP], ql[16 * KP];
    __shared__ __align__(16) _Float16 ks[KC * KP];
    __shared__ __align__(16) _Float16 vt[D * VP];
    __shared__ __align__(16) _Float16 ph[16 * VP], pl[16 * VP];
    __shared__ float sc[DH][16][KC];
    __shared__ float qscale[16], mrun[16], lrun[16], alpha[16];
    __shared__ int tok[16], lo_q[16], hi_q[16];

    const uint32_t tid = threadIdx.x, lane = tid & 63, wave = tid >> 6, m = lane & 15, kq = lane >> 4;
    const uint32_t c = blockIdx.x, h = blockIdx.y, qt = blockIdx.z;
    const uint32_t q_heads = a.kv_heads * a.group, nq = a.T * a.group;
    if (tid < 16) {
        const uint32_t qi = 16 * qt + tid;
        const bool ok = qi < nq;
        const int p = (int)(a.pos0 + (ok ? qi / a.group : 0));
        tok[tid] = ok ? (int)(qi / a.group) : -1;
        hi_q[tid] = ok ? p : -1;
        lo_q[tid] = a.window ? max(0, p + 1 - (int)a.window) : 0;
        mrun[tid] = -INFINITY;
        lrun[tid] = 0.0f;
    }
    // the tile's queries as scaled fp16 pairs (wave w: rows 4 w .. 4 w + 3)
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const uint32_t r = 4 * wave + i, qi = 16 * qt + r;
        float v[D / 64];
        const bool ok = qi < nq;
        const float* src = a.q + ((size_t)(ok ? qi / a.group : 0) * q_heads + h * a.group + qi % a.group) * D;
        float mx = 0.0f;
#pragma unroll
        for (int j = 0; j < D / 64; ++j) {
            v[j] = ok ? src[lane + 64 * j] : 0.0f;
            mx = fmaxf(mx, fabsf(v[j]));
        }
        mx = wave_max(mx);
        const float s = mx > 0.0f ? ldexpf(1.0f, 4 - ilogbf(mx)) : 1.0f;  // |q s| < 32
#pragma unroll
        for (int j = 0; j < D / 64; ++j) split_f16(v[j] * s, qh[r * KP + lane + 64 * j], ql[r * KP + lane + 64 * j]);
        if (lane == 0) qscale[r] = 1.0f / s;
    }
    const uint32_t k_begin = a.klo + c * a.span, k_end = min(k_begin + a.span, a.pos0 + a.T);
    v4f acc[NT];
#pragma unroll
    for (int j = 0; j < NT; ++j) acc[j] = v4f{0.0f, 0.0f, 0.0f, 0.0f};

    for (uint32_t k0 = k_begin; k0 < k_end; k0 += KC) {
        __syncthreads();  // the last sub-chunk's K, V^T, probabilities and alpha are read
        const uint32_t kn = min((uint32_t)KC, k_end - k0);
        for (uint32_t i = tid; i < KC * D / 8; i += 256) {  // K rows, 16-byte pieces
            const uint32_t row = i / (D / 8), pc = i % (D / 8);
            v4u val = {0u, 0u, 0u, 0u};
            if (row < kn) val = *gp(reinterpret_cast<const v4u*>(a.kcache + ((size_t)h * a.ring + (k0 + row) % a.ring) * D + 8 * pc));
            *reinterpret_cast<v4u*>(ks + row * KP + 8 * pc) = val;
        }
        for (uint32_t i = tid; i < KC / 2 * (D / 8); i += 256) {  // V rows 2j, 2j + 1 -> V^T
            const uint32_t j = i / (D / 8), pc = i % (D / 8);
            v4u v0 = {0u, 0u, 0u, 0u}, v1 = {0u, 0u, 0u, 0u};
            if (2 * j < kn)
                v0 = *gp(reinterpret_cast<const v4u*>(a.vcache + ((size_t)h * a.ring + (k0 + 2 * j) % a.ring) * D + 8 * pc));
            if (2 * j + 1 < kn)
                v1 = *gp(reinterpret_cast<const v4u*>(a.vcache + ((size_t)h * a.ring + (k0 + 2 * j + 1) % a.ring) * D + 8 * pc));
            const uint32_t w0[4] = {v0.x, v0.y, v0.z, v0.w}, w1[4] = {v1.x, v1.y, v1.z, v1.w};
#pragma unroll
            for (int e = 0; e < 8; ++e) {  // channel 8 pc + e: (key 2j, key 2j + 1)
                const uint32_t d = (e & 1) ? __builtin_amdgcn_perm(w1[e / 2], w0[e / 2], 0x07060302u)
                                           : __builtin_amdgcn_perm(w1[e / 2], w0[e / 2], 0x05040100u);
                *reinterpret_cast<uint32_t*>(vt + (8 * pc + e) * VP + 2 * j) = d;
            }
        }
        __syncthreads();
        {  // scores: wave w -> key tile w % KT, head-width part w / KT; lane: S[4 kq + i][16 kt + m]
            const uint32_t kt = wave % KT, dp = wave / KT;
            v4f sv = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
            for (int d = 0; d < DS; ++d) {
                const uint32_t k = 32 * (dp * DS + d) + 8 * kq;
                const v8h B = *reinterpret_cast<const v8h*>(ks + (16 * kt + m) * KP + k);
                sv = __builtin_amdgcn_mfma_f32_16x16x32_f16(*reinterpret_cast<const v8h*>(qh + m * KP + k), B, sv, 0, 0, 0);
                sv = __builtin_amdgcn_mfma_f32_16x16x32_f16(*reinterpret_cast<const v8h*>(ql + m * KP + k), B, sv, 0, 0, 0);
            }
#pragma unroll
            for (int i = 0; i < 4; ++i) sc[dp][4 * kq + i][16 * kt + m] = sv[i];
        }
        __syncthreads();
        // online softmax, wave w: queries 4 w .. 4 w + 3, lane = key
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const uint32_t r = 4 * wave + i, key = k0 + lane;
            float s = -INFINITY;
            if (lane < (uint32_t)KC && tok[r] >= 0 && key < k_end && (int)key >= lo_q[r] && (int)key <= hi_q[r]) {
                float v = sc[0][r][lane];
#pragma unroll
                for (int dp = 1; dp < DH; ++dp) v += sc[dp][r][lane];
                s = v * qscale[r] * a.scale;
            }
            const float mo = mrun[r], mn = fmaxf(mo, wave_max(s));
            const float p = s == -INFINITY ? 0.0f : expf(s - mn);
            const float al = mn == -INFINITY ? 1.0f : expf(mo - mn);
            const float sum = wave_sum(p);
            if (lane < (uint32_t)KC) split_f16(p * 16384.0f, ph[r * VP + lane], pl[r * VP + lane]);
            if (lane == 0) {
                mrun[r] = mn;
                lrun[r] = fmaf(lrun[r], al, sum);
                alpha[r] = al;
            }
        }
        __syncthreads();
        {  // values: wave w -> channel tiles w NT + j; lane: O[4 kq + i][16 (w NT + j) + m]
            float al[4];
#pragma unroll
            for (int i = 0; i < 4; ++i) al[i] = alpha[4 * kq + i];
#pragma unroll
            for (int j = 0; j < NT; ++j) {
#pragma unroll
                for (int i = 0; i < 4; ++i) acc[j][i] *= al[i];
                const uint32_t dim = 16 * (wave * NT + j) + m;
#pragma unroll
                for (int kk = 0; kk < KC / 32; ++kk) {
                    const uint32_t k = 32 * kk + 8 * kq;
                    const v8h B = *reinterpret_cast<const v8h*>(vt + dim * VP + k);
                    acc[j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(*reinterpret_cast<const v8h*>(ph + m * VP + k), B, acc[j], 0, 0, 0);
                    acc[j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(*reinterpret_cast<const v8h*>(pl + m * VP + k), B, acc[j], 0, 0, 0);
                }
            }
        }
    }
    __syncthreads();
    // chunk partials: sum p v (the probabilities' 2^14 removed), max, sum p
#pragma unroll
    for (int j = 0; j < NT; ++j)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const uint32_t r = 4 * kq + i;
            if (tok[r] < 0) continue;
            const uint32_t qi = 16 * qt + r, row = (uint32_t)tok[r] * q_heads + h * a.group + qi % a.group;
            a.part[((size_t)row * a.nchunks + c) * (D + 2) + 16 * (wave * NT + j) + m] = acc[j][i] * (1.0f / 16384.0f);
        }
    if (tid < 16 && tok[tid] >= 0) {
        const uint32_t qi = 16 * qt + tid, row = (uint32_t)tok[tid] * q_heads + h * a.group + qi % a.group;
        float* pr = a.part + ((size_t)row * a.nchunks + c) * (D + 2);
        pr[D] = mrun[tid];
        pr[D + 1] = lrun[tid];
    }
}

// out[t][qh] = sum_c w_c o_c / sum_c w_c l_c, w_c = exp(m_c - max_c m_c), chunks in order; one
// workgroup per (token, query head), one thread per channel.
template <int D>
__global__ __launch_bounds__(D) void batch_attention_merge_kernel(BatchAttn a) {
    const uint32_t row = blockIdx.x, q_heads = a.kv_heads * a.group, t = row / q_heads, qh = row % q_heads;
    const float* pr = a.part + (size_t)row * a.nchunks * (D + 2);
    float M = -INFINITY;
    for (uint32_t c = 0; c < a.nchunks; ++c) M = fmaxf(M, pr[c * (D + 2) + D]);
    float L = 0.0f, acc = 0.0f;
    for (uint32_t c = 0; c < a.nchunks; ++c) {
        const float mc = pr[c * (D + 2) + D];
        const float w = mc == -INFINITY ? 0.0f : expf(mc - M);
        L = fmaf(w, pr[c * (D + 2) + D + 1], L);
        acc = fmaf(w, pr[c * (D + 2) + threadIdx.x], acc);
    }
    a.out[(size_t)t * a.out_stride + (size_t)qh * D + threadIdx.x] = acc / L;
}

// ---- launchers ----------------------------------------------------------------------------------

// Chunks of the batch's key range: about one per 64 keys, at most kBatchAttnChunks (a chunk then
// spans several sub-chunks).
hipError_t launch_batch_attention(BatchAttn a, uint32_t head_width, hipStream_t s) {
    if (a.T == 0 || a.T > kBatchMax || a.kv_heads == 0 || a.group == 0) return hipErrorInvalidValue;
    const uint32_t KC = head_width == 256 ? 64 : 32;
    const int64_t lo = a.window ? std::max<int64_t>(0, (int64_t)a.pos0 + 1 - a.window) : 0;
    const uint32_t keys = a.pos0 + a.T - (uint32_t)lo;
    const uint32_t sub = (keys + KC - 1) / KC;
    const uint32_t per = (sub + kBatchAttnChunks - 1) / kBatchAttnChunks;
    a.klo = (uint32_t)lo;
    a.span = per * KC;
    a.nchunks = (keys + a.span - 1) / a.span;
    const uint32_t tiles = (a.T * a.group + 15) / 16;
    const dim3 grid(a.nchunks, a.kv_heads, tiles);
    if (head_width == 256) {
        hipLaunchKernelGGL((batch_attention_kernel<256, 64>), grid, dim3(256), 0, s, a);
        if (hipGetLastError() != hipSuccess) return hipErrorLaunchFailure;
        hipLaunchKernelGGL((batch_attention_merge_kernel<256>), dim3(a.T * a.kv_heads * a.group), dim3(256), 0, s, a);
    } else if (head_width == 512) {
        hipLaunchKernelGGL((batch_attention_kernel<512, 32>), grid, dim3(256), 0, s, a);
        if (hipGetLastError() != hipSuccess) return hipErrorLaunchFailure;
        hipLaunchKernelGGL((batch_attention_merge_kernel<512>), dim3(a.T * a.kv_heads * a.group), dim3(512), 0, s, a);
    } else {
        return hipErrorInvalidValue;
    }
    return hipGetLastError();
}


size_t batch_image_bytes(uint32_t blocks, uint32_t tokens) {
    return (size_t)blocks * padded_tokens(tokens) * (128 + 4);
}

size_t batch_gemm_part_bytes(uint32_t rows, uint32_t blocks, uint32_t tokens, bool gelu_pair) {
    const GemmPlan p = gemm_plan(rows, blocks, gelu_pair);
    if (p.S == 1) return 0;
    return (size_t)p.S * (gelu_pair ? 2 : 1) * padded_tokens(tokens) * ((rows + 15) / 16 * 16) * 4;
}

hipError_t launch_batch_input(const BatchIn& in, hipStream_t s) {
    if (in.T == 0 || in.T > kBatchMax || in.K == 0 || in.K > 16384 || in.K % 32) return hipErrorInvalidValue;
    if (in.mode == BI_PLAIN && !in.w_n) {
        if (in.stride % 4 || reinterpret_cast<uintptr_t>(in.x) % 16) return hipErrorInvalidValue;
        const uint32_t octets = in.K / 8;
        const dim3 g(padded_tokens(in.T), (octets + 255) / 256);
        if (in.parts) {
            if (in.parts > kDeferPairParts || reinterpret_cast<uintptr_t>(in.part) % 16 || in.part_row % 4 ||
                in.part_row < in.K)
                return hipErrorInvalidValue;
            hipLaunchKernelGGL(batch_plain_input_kernel<true>, g, dim3(256), 0, s, in);
        } else {
            hipLaunchKernelGGL(batch_plain_input_kernel<false>, g, dim3(256), 0, s, in);
        }
    } else {
        // float4 access to x, res, x_out and the norm weights
        const auto a16 = [](const void* p) { return reinterpret_cast<uintptr_t>(p) % 16 == 0; };
        if (in.stride % 4 || !a16(in.x) || !a16(in.res) || !a16(in.x_out) || !a16(in.w_a) || !a16(in.w_n))
            return hipErrorInvalidValue;
        const uint32_t octets = in.K / 8;
        const dim3 g(padded_tokens(in.T));
        const size_t lds = in.mode == BI_EMBED ? (size_t)in.K * 4 : 0;
        if (in.parts) {
            if (in.mode != BI_RESID || octets > 512 || in.parts > kDeferParts || !a16(in.part) || in.part_row % 4 ||
                in.part_row < in.K)
                return hipErrorInvalidValue;
            hipLaunchKernelGGL((batch_input_kernel<1, true>), g, dim3(512), 0, s, in);
        } else if (octets <= 512) {
            hipLaunchKernelGGL((batch_input_kernel<1, false>), g, dim3(512), lds, s, in);
        } else if (octets <= 1024) {
            hipLaunchKernelGGL((batch_input_kernel<2, false>), g, dim3(512), lds, s, in);
        } else {
            hipLaunchKernelGGL((batch_input_kernel<4, false>), g, dim3(512), lds, s, in);
        }
    }
    return hipGetLastError();
}

template <int P, int G>
static hipError_t gemm_launch(const BatchGemm& a, hipStream_t s, uint32_t* parts) {
    const GemmPlan p = gemm_plan(a.w.rows, a.w.blocks, P == 2);
    const uint32_t tiles = (a.w.rows + 15) / 16;
    const dim3 grid((tiles + p.R - 1) / p.R, p.S);
    if (p.S > 1 && !a.part) return hipErrorInvalidValue;
    switch (p.R) {
        case 1: hipLaunchKernelGGL((batch_gemm_kernel<P, G, 1>), grid, dim3(kGemmThreads), 0, s, a); break;
        case 2: hipLaunchKernelGGL((batch_gemm_kernel<P, G, 2>), grid, dim3(kGemmThreads), 0, s, a); break;
        case 4: hipLaunchKernelGGL((batch_gemm_kernel<P, G, 4>), grid, dim3(kGemmThreads), 0, s, a); break;
        default:
            if constexpr (P == 1) hipLaunchKernelGGL((batch_gemm_kernel<P, G, 8>), grid, dim3(kGemmThreads), 0, s, a);
            break;
    }
    hipError_t e = hipGetLastError();
    if (e != hipSuccess || p.S == 1) return e;
    if (a.defer && !a.add && p.S <= (P == 2 ? kDeferPairParts : kDeferParts)) {
        if (parts) *parts = p.S;
        return hipSuccess;
    }
    const uint32_t n = a.T * a.w.rows;
    hipLaunchKernelGGL((batch_reduce_kernel<P>), dim3((n + 255) / 256), dim3(256), 0, s, a, p.S, 16u * G);
    return hipGetLastError();
}

hipError_t launch_batch_gemm(const BatchGemm& a, bool gelu_pair, hipStream_t s, uint32_t* parts) {
    if (parts) *parts = 0;
    if (a.T == 0 || a.T > kBatchMax || a.w.rows == 0 || a.w.blocks == 0) return hipErrorInvalidValue;
    if (gelu_pair && (a.w2.rows != a.w.rows || a.w2.blocks != a.w.blocks)) return hipErrorInvalidValue;
    const bool two = a.T > 16;
    if (gelu_pair) return two ? gemm_launch<2, 2>(a, s, parts) : gemm_launch<2, 1>(a, s, parts);
    return two ? gemm_launch<1, 2>(a, s, parts) : gemm_launch<1, 1>(a, s, parts);
}

}  // namespace af
