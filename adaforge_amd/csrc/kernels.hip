// HIP kernels for gfx950 (MI355X): the per-operation entry points of the decode step of a
// Q4_0 / Q6_K transformer (Q4_0 GEMV on the int8 matrix cores, Q6_K head with greedy argmax,
// GQA decode attention, RMSNorm).  Cross-workgroup results (attention chunks, argmax
// partials) are combined by the last workgroup to finish, found with a device-scope counter
// that the last workgroup resets, so the kernels can be replayed in a graph.
#include "device.h"

namespace af {

// Cross-workgroup partials (argmax, attention chunks) are combined by the last workgroup to finish.
// The workgroups run on all 8 XCDs, whose L2s are not coherent with each other, so the partials
// are stored through to the memory side (policy sc1) and waited for before an agent-scope ticket,
// and the last workgroup reads them from the memory side: no device-scope fence, which would write
// back and invalidate the L2.
constexpr int kPartSC1 = 16;       // buffer access policy sc1: through to (or from) the memory side
constexpr int kPartSC0 = 1;        // stores: workgroup scope, into the XCD's L2
constexpr int kPartNT = 2;         // loads: non-temporal, miss the CU's L1 and hit the XCD's L2
constexpr int kWaitVm0 = 0x0F70;   // s_waitcnt vmcnt(0), expcnt and lgkmcnt unconstrained

// ---- Q4_0 GEMV: persistent, one workgroup per CU ----------------------------------------------
//
// The output rows come in units of one 16-row tile (T = 2: the same tile of the gate and the up
// matrix), taken in groups of UG consecutive units: workgroup b takes groups b, b + G, ... (G = grid
// size).  UG = 2 (UGS = 1) when the GELU epilogue also writes the digit image of its output (a.dig_out, the
// next GEMV's IN_DIGITS input), so that every 32-element block of it belongs to one workgroup.  The
// super-tiles of a workgroup's units,
// flattened in (unit, matrix, super-tile) order, are dealt round-robin to its 8 waves, so every
// wave streams one sequence of records across tile boundaries.  Each wave keeps kGemvRing records
// in flight in registers: it folds a record, then requests the one kGemvRing places further on,
// with the same two load instructions whether that record exists or not (past the end the
// buffer's range is 0 and the load returns zeros without a memory access), so the compiler's
// wait for each record is an exact count.  The first records are requested before the prologue
// builds the input's digit image, which thus runs while they are in flight.  A wave adds each
// tile's row sums to LDS once, when its records move on to the next tile; the epilogue adds the
// 8 waves' partials of a row in wave order.
constexpr int kGemvRing = 8;             // records in flight per wave
constexpr uint32_t kGemvMaxUnits = 8;    // units per workgroup (more units: a larger grid)
constexpr uint32_t kGemvWaves = 8;

struct GemvCursor {
    uint32_t j, k, st;  // unit of the workgroup, matrix, super-tile (wave-uniform)
};

__device__ __forceinline__ void gemv_advance(GemvCursor& c, uint32_t nst, uint32_t T) {
    c.st += kGemvWaves;
    while (c.st >= nst) {
        c.st -= nst;
        if (++c.k == T) {
            c.k = 0;
            ++c.j;
        }
    }
}

template <int T, int IN, int OUT, int Q, int UGS>
__global__ __launch_bounds__(512) void q4_gemv_kernel(Q4Args a, uint32_t out_rows, uint32_t units) {
    constexpr uint32_t ugs = UGS;
    extern __shared__ __align__(16) uint8_t smem[];
    __shared__ double red[16];
    __shared__ float part[kGemvWaves][kGemvMaxUnits * T][16];

    if (a.state && a.state[ST_STOP]) return;
    const uint32_t tid = threadIdx.x, lane = tid & 63, wave = wave_id();
    const uint32_t G = gridDim.x, b = blockIdx.x;
    const uint32_t B = a.w.blocks, K = B * 32, nst = a.w.nst;
    // groups of UG = 2^UGS units: the grid never exceeds the groups, and UG divides the units
    const uint32_t nu = ((units >> ugs) - b + G - 1) / G << ugs;
    auto unit_of = [&](uint32_t j) { return ((b + (j >> ugs) * G) << ugs) + (j & ((1u << ugs) - 1)); };
    const uint32_t N = nu * T * nst;               // records of this workgroup
    const uint32_t n_w = N > wave ? (N - wave + kGemvWaves - 1) / kGemvWaves : 0;

    // record r = wave + 8 i of the workgroup's sequence
    GemvCursor ld{0, 0, wave};
    while (ld.st >= nst) {  // more waves than one tile's super-tiles
        ld.st -= nst;
        if (++ld.k == (uint32_t)T) {
            ld.k = 0;
            ++ld.j;
        }
    }
    GemvCursor cs = ld;
    const uint32_t code_off = lane * 16, scale_off = lane * 2;
    v4u rc[kGemvRing];
    uint32_t rsc[kGemvRing];
    auto request = [&](int u, const GemvCursor& c, bool ok) {
        const bool second = T == 2 && c.k == 1;
        const uint8_t* codes = second ? a.w2.codes : a.w.codes;
        const uint16_t* scales = second ? a.w2.scales : a.w.scales;
        const size_t rec = (size_t)unit_of(c.j) * nst + c.st;
        const __amdgpu_buffer_rsrc_t rcode =
            __builtin_amdgcn_make_buffer_rsrc(const_cast<uint8_t*>(codes) + rec * 1024, 0, ok ? 1024 : 0, 0x00020000);
        const __amdgpu_buffer_rsrc_t rscale =
            __builtin_amdgcn_make_buffer_rsrc(const_cast<uint16_t*>(scales) + rec * 64, 0, ok ? 128 : 0, 0x00020000);
        rc[u] = __builtin_amdgcn_raw_buffer_load_b128(rcode, code_off, 0, 2);
        rsc[u] = __builtin_amdgcn_raw_buffer_load_b16(rscale, scale_off, 0, 2);
    };

    InputRegs<IN, Q> g;
    input_load<IN, Q>(a.in, K, nst, g);  // inputs first (see input_load)
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int u = 0; u < kGemvRing; ++u) {
        request(u, ld, (uint32_t)u < n_w);
        gemv_advance(ld, nst, T);
    }
    __builtin_amdgcn_sched_barrier(0);

    const size_t xs_bytes = IN == IN_EMBED ? (size_t)K * 4 : 0;
    int8_t* dig = reinterpret_cast<int8_t*>(smem + xs_bytes);
    BlockTab* tab = reinterpret_cast<BlockTab*>(smem + xs_bytes + (size_t)nst * 512);
    uint4* zero_blk = reinterpret_cast<uint4*>(smem + xs_bytes + (size_t)nst * kStepImg);  // 32 bytes
    input_digits<IN, Q>(a.in, K, nst, g, reinterpret_cast<float*>(smem), dig, tab, red);
    if (tid < 2) zero_blk[tid] = make_uint4(0u, 0u, 0u, 0u);
    float* pflat = &part[0][0][0];
    for (uint32_t i = tid; i < kGemvWaves * kGemvMaxUnits * T * 16; i += blockDim.x) pflat[i] = 0.0f;
    __syncthreads();

    // lane 16 q + r: A row r (digit plane r of the super-tile) in k-group q, which is non-zero when
    // r / 4 == q (the plane at a_base + st * a_step, else the zero block with a_step 0); D column r
    const uint32_t r = lane & 15, q = lane >> 4;
    const bool aon = (r >> 2) == q;
    const int8_t* a_base = aon ? dig + r * 32 : reinterpret_cast<const int8_t*>(zero_blk);
    const uint32_t a_step = aon ? 512u : 0u;
    float acc = 0.0f;
    uint32_t cur = cs.j * T + cs.k;
    auto flush = [&]() {
        acc = row_total(acc);  // row r over the 4 blocks (k-groups)
        if (q == 0) part[wave][cur][r] = acc;
        acc = 0.0f;
    };
    for (uint32_t i0 = 0; i0 < n_w; i0 += kGemvRing) {
#pragma unroll
        for (int u = 0; u < kGemvRing; ++u) {
            const uint32_t i = i0 + u;
            if (i < n_w) {
                const uint32_t sl = cs.j * T + cs.k;
                if (sl != cur) {
                    flush();
                    cur = sl;
                }
                const Q4Tile w{make_uint4(rc[u].x, rc[u].y, rc[u].z, rc[u].w), rsc[u]};
                const v4i* ap = reinterpret_cast<const v4i*>(a_base + cs.st * a_step);
                q4_mfma_tile(w, ap[0], ap[1], tab[cs.st * 4 + q], acc);
                gemv_advance(cs, nst, T);
            }
            request(u, ld, i + kGemvRing < n_w);
            gemv_advance(ld, nst, T);
        }
    }
    if (n_w > 0) flush();
    __syncthreads();
    const double rn = gemv_row_factor<IN>(red, K, a.in.eps_n);  // the input's deferred RMSNorm factor

    if constexpr (OUT == OUT_GELU) {
        if constexpr (UGS == 1) {  // the rows' GELU products, one per thread, then a digit block per 32-row group
            __shared__ float act_l[kGemvMaxUnits * 16];
            for (uint32_t i = tid; i < nu * 16; i += blockDim.x) {
                const uint32_t j = i >> 4, r = i & 15;
                float gs = part[0][j * T][r], us = part[0][j * T + 1][r];
                for (uint32_t w = 1; w < kGemvWaves; ++w) {
                    gs += part[w][j * T][r];
                    us += part[w][j * T + 1][r];
                }
                const float v = gelu_mul((float)(rn * (double)gs), (float)(rn * (double)us));
                act_l[i] = v;
                a.y[unit_of(j) * 16 + r] = v;
            }
            __syncthreads();
            int8_t* img = a.dig_out;
            BlockTab* otab = reinterpret_cast<BlockTab*>(img + (size_t)(out_rows / 128 + (out_rows % 128 != 0)) * 512);
            for (uint32_t i = tid; i < nu / 2 * 4; i += blockDim.x) {  // quads: 8 rows each of a group's 32
                const uint32_t jg = i >> 2, p = i & 3, blk = b + jg * G;
                float v[8];
#pragma unroll
                for (int e = 0; e < 8; ++e) v[e] = act_l[jg * 32 + 8 * p + e];
                float m, sum;
                quad_stats(v, m, sum);
                digits8(v, m, img, blk, p);
                if (p == 0) otab[blk] = block_tab(m, sum);
            }
            return;
        }
    }
    for (uint32_t i = tid; i < nu * 16; i += blockDim.x) {
        const uint32_t j = i >> 4, r = i & 15, row = unit_of(j) * 16 + r;
        if (row >= out_rows) continue;
        float v[T];
#pragma unroll
        for (int k = 0; k < T; ++k) {
            float s = part[0][j * T + k][r];
            for (uint32_t w = 1; w < kGemvWaves; ++w) s += part[w][j * T + k][r];
            v[k] = (float)(rn * (double)s);
        }
        if constexpr (OUT == OUT_GELU) a.y[row] = gelu_mul(v[0], v[T - 1]);
        else if constexpr (OUT == OUT_ADD) a.y[row] = __fadd_rn(v[0], a.add[row]);
        else a.y[row] = v[0];
    }
}

constexpr uint32_t kQ4Threads = 512;

// One workgroup per CU, more when the groups would exceed kGemvMaxUnits units per workgroup.
static uint32_t gemv_grid(uint32_t groups, uint32_t ug) {
    int dev = 0, cus = 256;
    if (hipGetDevice(&dev) != hipSuccess || hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess)
        cus = 256;
    const uint32_t per = kGemvMaxUnits / ug, need = (groups + per - 1) / per;
    return min(groups, max((uint32_t)cus, need));
}

template <int T, int IN, int OUT, int Q>
static hipError_t q4_launch3(Q4Args a, uint32_t out_rows, hipStream_t st) {
    const uint32_t units = (out_rows + 15) / 16;
    if (units == 0) return hipSuccess;
    a.slices = kGemvWaves;
    const size_t lds = (IN == IN_EMBED ? (size_t)a.w.blocks * 32 * 4 : 0) + (size_t)a.w.nst * kStepImg + 32;
    if constexpr (OUT == OUT_GELU) {
        if (a.dig_out) {  // a digit image of the output needs whole 32-row blocks per workgroup
            if (out_rows % 32) return hipErrorInvalidValue;
            hipLaunchKernelGGL((q4_gemv_kernel<T, IN, OUT, Q, 1>), dim3(gemv_grid(units / 2, 2)), dim3(kQ4Threads), lds,
                               st, a, out_rows, units);
            return hipGetLastError();
        }
    }
    hipLaunchKernelGGL((q4_gemv_kernel<T, IN, OUT, Q, 0>), dim3(gemv_grid(units, 1)), dim3(kQ4Threads), lds, st, a,
                       out_rows, units);
    return hipGetLastError();
}

// Octets per thread: the prologue covers 16 nst octets (128 nst elements) with 512 threads.
template <int T, int IN, int OUT>
static hipError_t q4_launch2(const Q4Args& a, uint32_t out_rows, hipStream_t st) {
    const uint32_t oct = a.w.nst * 16;
    if (oct <= kQ4Threads) return q4_launch3<T, IN, OUT, 1>(a, out_rows, st);
    if (oct <= 2 * kQ4Threads) return q4_launch3<T, IN, OUT, 2>(a, out_rows, st);
    return q4_launch3<T, IN, OUT, 4>(a, out_rows, st);
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
        case IN_DIGITS: return q4_launch1<IN_DIGITS>(a, out_kind, out_rows, s);
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

// ---- Q6_K head on the int8 matrix cores --------------------------------------------------------
//
// The table is read as records of 16 rows x one 256-weight super-block (Q6View::t, kQ6Rec bytes,
// built at upload).  Per record, four v_mfma_i32_16x16x64_i8 over its 64-weight k-blocks: A = the
// input's digit planes (row 4 g + t: digit t of 16-element group g; the 16 lanes whose k-group is
// g read them, the others a zero block), B = the codes of (group g, row r) at lane 16 g + r, as
// the lane's 16 unsigned 6-bit codes.  Lane 16 g + r then holds D[4 g + t][r] for t = 0..3, which
// it folds with the group's plane scales and its sub-block scale, and with the row's d once per
// record.  Input x_j ~ s (q0 + q1 2^-7 + q2 2^-14 + q3 2^-21) per 16-element group (s = 2^(e - 5),
// e = ilogb of the group's max |x|): exact for |x_j| >= 2^(e - 3), otherwise within 2^(e - 27).

constexpr int kHeadRing = 4;  // records in flight per wave (4, 6 and 8 within 1.3 % of one another)

// A wave's head state: its ring of records and its position in its tile sequence.
struct HeadRing {
    v4u code[kHeadRing][3];  // the lane's 12 code dwords per record (3 per k-block)
    uint32_t sc[kHeadRing];  // the lane's 4 sub-block scales (int8, one per k-block)
    uint32_t d[kHeadRing];   // the lane's row d (fp16 in the low half)
};

// 16 unsigned 6-bit codes from a lane's dwords L0, L1 (low nibbles of codes b and 4 + b in byte b,
// and of codes 8 + b, 12 + b) and H (high bit pairs of codes b, 4 + b, 8 + b, 12 + b in byte b).
__device__ __forceinline__ v4i q6_unpack(uint32_t l0, uint32_t l1, uint32_t h) {
    constexpr uint32_t M = 0x0F0F0F0Fu, M3 = 0x30303030u;
    return v4i{(int)((l0 & M) | ((h << 4) & M3)), (int)(((l0 >> 4) & M) | ((h << 2) & M3)),
               (int)((l1 & M) | (h & M3)), (int)(((l1 >> 4) & M) | ((h >> 2) & M3))};
}

__device__ __forceinline__ void head_fill(HeadRing& hr, int u, const __amdgpu_buffer_rsrc_t& rs, uint32_t rec,
                                          uint32_t lane) {
    const int off = (int)(rec * kQ6Rec);
#pragma unroll
    for (int p = 0; p < 3; ++p) hr.code[u][p] = __builtin_amdgcn_raw_buffer_load_b128(rs, p * 1024 + lane * 16, off, 2);
    hr.sc[u] = __builtin_amdgcn_raw_buffer_load_b32(rs, 3072 + lane * 4, off, 2);
    hr.d[u] = __builtin_amdgcn_raw_buffer_load_b16(rs, 3328 + (lane & 15) * 2, off, 2);
}

template <int IN>
__global__ __launch_bounds__(512) void q6_head_kernel(HeadArgs a) {
    extern __shared__ __align__(16) uint8_t hl[];  // xs [K] f32, digit planes [K / 16][4][16], tab [K / 16]
    __shared__ double red[16];
    __shared__ float wv[8];
    __shared__ uint32_t wi[8], wb[8];
    __shared__ bool last;
    __shared__ uint4 zero_blk[2];

    if (a.state && a.state[ST_STOP]) return;
    const uint32_t K = a.w.units * 64, sb = K / 256, rows = a.w.rows, ntiles = (rows + 15) / 16;
    const uint32_t tid = threadIdx.x, lane = tid & 63, wave = wave_id();
    const uint32_t nw = gridDim.x * (blockDim.x / 64), gw = blockIdx.x * (blockDim.x / 64) + wave;
    float* xs = reinterpret_cast<float*>(hl);
    uint8_t* dig = hl + (size_t)K * 4;
    float4* tab = reinterpret_cast<float4*>(dig + (size_t)K * 4);
    if (tid < 2) zero_blk[tid] = make_uint4(0u, 0u, 0u, 0u);

    // the wave's records: tiles gw, gw + nw, ... below ntiles, sb records each
    const uint32_t my_tiles = gw < ntiles ? (ntiles - gw + nw - 1) / nw : 0;
    const uint32_t total = my_tiles * sb;
    const __amdgpu_buffer_rsrc_t rs =
        __builtin_amdgcn_make_buffer_rsrc(const_cast<uint8_t*>(a.w.t), 0, (int)(ntiles * sb * kQ6Rec), 0x00020000);
    HeadRing hr;
    uint32_t ft = gw, fs = 0;  // next record to request: tile ft, super-block fs (past the end: record 0)
    auto fill = [&](int u) {
        const uint32_t rec = ft < ntiles ? ft * sb + fs : 0u;
        head_fill(hr, u, rs, rec, lane);
        if (++fs == sb) {
            fs = 0;
            ft += nw;
        }
    };
#pragma unroll
    for (int u = 0; u < kHeadRing; ++u) fill(u);  // weights first: their latency overlaps the input stage

    if constexpr (IN == IN_PLAIN) {
        const float4* src = reinterpret_cast<const float4*>(a.in.x);
        float4* dst = reinterpret_cast<float4*>(xs);
        for (uint32_t i = tid; i < K / 4; i += blockDim.x) dst[i] = src[i];
        __syncthreads();
    } else {
        input_stage<IN>(a.in, xs, K, red);
    }
    // digit image: thread i < K / 16 takes group i
    if (tid < K / 16) {
        float v0[8], v1[8], m = 0.0f, sum = 0.0f;
#pragma unroll
        for (int k = 0; k < 8; ++k) {
            v0[k] = xs[16 * tid + k];
            v1[k] = xs[16 * tid + 8 + k];
            m = fmaxf(m, fmaxf(fabsf(v0[k]), fabsf(v1[k])));
            sum += v0[k] + v1[k];
        }
        uint32_t w0[4][2], w1[4][2];
        digit_words(v0, m, w0);
        digit_words(v1, m, w1);
#pragma unroll
        for (int t = 0; t < 4; ++t)
            reinterpret_cast<uint4*>(dig)[tid * 4 + t] = make_uint4(w0[t][0], w0[t][1], w1[t][0], w1[t][1]);
        const float sc = m > 0.0f ? ldexpf(1.0f, ilogbf(m) - 5) : 0.0f;
        tab[tid] = make_float4(ldexpf(sc, -14), ldexpf(sc, -21), -32.0f * sum, 0.0f);
    }
    __syncthreads();

    const uint32_t g = lane >> 4, r = lane & 15;
    const bool aon = (r >> 2) == g;
    const uint32_t a0 = aon ? lds_addr(dig) + r * 16 : lds_addr(zero_blk), am = aon ? 256u : 0u;
    const uint32_t t0 = lds_addr(tab) + g * 16;
    float bv = -INFINITY, acc = 0.0f;
    uint32_t bi = 0xFFFFFFFFu, bad = 0;
    uint32_t ct = gw, cs = 0;  // record being consumed
    auto record = [&](int u) {
        float sbacc = 0.0f;
#pragma unroll
        for (int kb = 0; kb < 4; ++kb) {
            const uint32_t wl0 = hr.code[u][(3 * kb) / 4][(3 * kb) % 4];
            const uint32_t wl1 = hr.code[u][(3 * kb + 1) / 4][(3 * kb + 1) % 4];
            const uint32_t wh = hr.code[u][(3 * kb + 2) / 4][(3 * kb + 2) % 4];
            const uint32_t blk = cs * 4 + kb;  // k-block of the row
            const v4i av = lds_at<v4i>(a0 + blk * am);
            const v4i d = __builtin_amdgcn_mfma_i32_16x16x64_i8(av, q6_unpack(wl0, wl1, wh), v4i{0, 0, 0, 0}, 0, 0, 0);
            const v4f tb = lds_at<v4f>(t0 + blk * 64);
            // 2^14 D0 + 2^7 D1 + D2 is exact in int32 (|D_t| <= 16 * 63 * 64)
            const int I = (d[0] << 14) + (d[1] << 7) + d[2];
            float in = fmaf((float)I, tb.x, tb.z);
            in = fmaf((float)d[3], tb.y, in);
            sbacc = fmaf((float)(int8_t)(hr.sc[u] >> (8 * kb)), in, sbacc);
        }
        acc = fmaf(h2f((uint16_t)hr.d[u]), sbacc, acc);
        fill(u);  // after the last use of the slot's registers
        if (++cs == sb) {  // the tile's last record: its 16 rows
            const float v = row_total(acc);
            acc = 0.0f;
            const uint32_t row = ct * 16 + r;
            if (lane < 16 && row < rows) {
                if (a.logits) a.logits[row] = v;
                if (!isfinite(v)) bad = 1;
                else if (better(v, row, bv, bi)) {
                    bv = v;
                    bi = row;
                }
            }
            cs = 0;
            ct += nw;
        }
    };
    for (uint32_t i = total / kHeadRing; i; --i) {
#pragma unroll
        for (int u = 0; u < kHeadRing; ++u) record(u);
    }
    const uint32_t rem = total % kHeadRing;
#pragma unroll
    for (int u = 0; u < kHeadRing - 1; ++u)
        if ((uint32_t)u < rem) record(u);
    __builtin_amdgcn_s_waitcnt(0x0F70);  // the ring's last requests (past the end) before exit

    // wave, then workgroup, then grid: the greatest value, smallest id on ties, any non-finite
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
        const float ov = __shfl_xor(bv, o);
        const uint32_t oi = __shfl_xor(bi, o);
        if (better(ov, oi, bv, bi)) {
            bv = ov;
            bi = oi;
        }
        bad |= __shfl_xor(bad, o);
    }
    if (lane == 0) {
        wv[wave] = bv;
        wi[wave] = bi;
        wb[wave] = bad;
    }
    __syncthreads();
    if (threadIdx.x == 0) {
        for (uint32_t w = 1; w < blockDim.x / 64; ++w) {
            if (better(wv[w], wi[w], bv, bi)) {
                bv = wv[w];
                bi = wi[w];
            }
            bad |= wb[w];
        }
        __builtin_amdgcn_raw_buffer_store_b128(v4u{__float_as_uint(bv), bi, bad, 0u},
                                               __builtin_amdgcn_make_buffer_rsrc(a.partial, 0, 0x7FFFFFFF, 0x00020000),
                                               blockIdx.x * 16, 0, kPartSC1);
        __builtin_amdgcn_s_waitcnt(kWaitVm0);
        const uint32_t ticket = __hip_atomic_fetch_add(a.counter, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        last = ticket == gridDim.x - 1;
    }
    __syncthreads();
    if (!last) return;
    const __amdgpu_buffer_rsrc_t prs = __builtin_amdgcn_make_buffer_rsrc(a.partial, 0, 0x7FFFFFFF, 0x00020000);
    float v = -INFINITY;
    uint32_t id = 0xFFFFFFFFu, flag = 0;
    for (uint32_t b = threadIdx.x; b < gridDim.x; b += blockDim.x) {
        const v4u p = __builtin_amdgcn_raw_buffer_load_b128(prs, b * 16, 0, kPartSC1);
        const float pv = __uint_as_float(p.x);
        if (better(pv, p.y, v, id)) {
            v = pv;
            id = p.y;
        }
        flag |= p.z;
    }
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
        const float ov = __shfl_xor(v, o);
        const uint32_t oi = __shfl_xor(id, o);
        if (better(ov, oi, v, id)) {
            v = ov;
            id = oi;
        }
        flag |= __shfl_xor(flag, o);
    }
    if (lane == 0) {
        wv[wave] = v;
        wi[wave] = id;
        wb[wave] = flag;
    }
    __syncthreads();
    if (threadIdx.x == 0) {
        for (uint32_t w = 1; w < blockDim.x / 64; ++w) {
            if (better(wv[w], wi[w], v, id)) {
                v = wv[w];
                id = wi[w];
            }
            flag |= wb[w];
        }
        const uint32_t best = id, flagged = flag || best >= rows;
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
                StepRecord rc;
                rc.id = best;
                rc.bad = flagged;
                rc.stop = stop;
                rc.done = 1u;
                a.records[pos + 1] = rc;
            }
        }
        __hip_atomic_store(a.counter, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
}

// One workgroup of 8 waves per CU (at most), each wave striding over 16-row tiles.
uint32_t head_grid(uint32_t rows) {
    const uint32_t tiles = (rows + 15) / 16;
    const uint32_t g = (tiles + 7) / 8;
    return g > 256 ? 256 : g;
}

hipError_t launch_head(const HeadArgs& a, int in_kind, uint32_t grid, hipStream_t s) {
    const size_t K = (size_t)a.w.units * 64, lds = K * 4 + K * 4 + K;  // xs, digit planes, tab
    switch (in_kind) {
        case IN_PLAIN: hipLaunchKernelGGL(q6_head_kernel<IN_PLAIN>, dim3(grid), dim3(512), lds, s, a); break;
        case IN_NORM: hipLaunchKernelGGL(q6_head_kernel<IN_NORM>, dim3(grid), dim3(512), lds, s, a); break;
        case IN_RESID: hipLaunchKernelGGL(q6_head_kernel<IN_RESID>, dim3(grid), dim3(512), lds, s, a); break;
        default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

// ---- the head over several hidden states (speculative verification) ----------------------------
//
// q6_head_kernel's record loop with NV input vectors: vector v is a.in with x and res advanced by
// v vstride floats (the batched layers' rows), the same norms, no residual output and no logits.
// The table is read once: each record's codes are unpacked once and fed to one MFMA per vector
// and k-block.  Vector v's greedy id and non-finite flag go to a.result[2 v], a.result[2 v + 1].
// LDS: xs [K] f32 (each vector's input stage in turn), then per vector its digit planes
// [K / 16][4][16] and table [K / 16].  a.partial holds NV entries per workgroup.
template <int NV>
__global__ __launch_bounds__(512) void q6_head_batch_kernel(HeadArgs a, uint32_t vstride) {
    extern __shared__ __align__(16) uint8_t hl[];
    __shared__ double red[16];
    __shared__ float wv[8][NV];
    __shared__ uint32_t wi[8][NV], wb[8][NV];
    __shared__ bool last;
    __shared__ uint4 zero_blk[2];

    const uint32_t K = a.w.units * 64, sb = K / 256, rows = a.w.rows, ntiles = (rows + 15) / 16;
    const uint32_t tid = threadIdx.x, lane = tid & 63, wave = wave_id();
    const uint32_t nw = gridDim.x * (blockDim.x / 64), gw = blockIdx.x * (blockDim.x / 64) + wave;
    float* xs = reinterpret_cast<float*>(hl);
    uint8_t* const img0 = hl + (size_t)K * 4;  // vector v: digits at img0 + v 5K, table 4K after them
    if (tid < 2) zero_blk[tid] = make_uint4(0u, 0u, 0u, 0u);

    const uint32_t my_tiles = gw < ntiles ? (ntiles - gw + nw - 1) / nw : 0;
    const uint32_t total = my_tiles * sb;
    const __amdgpu_buffer_rsrc_t rs =
        __builtin_amdgcn_make_buffer_rsrc(const_cast<uint8_t*>(a.w.t), 0, (int)(ntiles * sb * kQ6Rec), 0x00020000);
    HeadRing hr;
    uint32_t ft = gw, fs = 0;
    auto fill = [&](int u) {
        const uint32_t rec = ft < ntiles ? ft * sb + fs : 0u;
        head_fill(hr, u, rs, rec, lane);
        if (++fs == sb) {
            fs = 0;
            ft += nw;
        }
    };
#pragma unroll
    for (int u = 0; u < kHeadRing; ++u) fill(u);  // weights first: their latency overlaps the input stages

#pragma unroll 1
    for (int v = 0; v < NV; ++v) {
        InputStage in = a.in;
        in.x += (size_t)v * vstride;
        in.res += (size_t)v * vstride;
        in.x_out = nullptr;
        input_stage<IN_RESID>(in, xs, K, red);
        uint8_t* dig = img0 + (size_t)v * 5 * K;
        float4* tab = reinterpret_cast<float4*>(dig + (size_t)K * 4);
        if (tid < K / 16) {  // thread i takes group i (as q6_head_kernel)
            float v0[8], v1[8], m = 0.0f, sum = 0.0f;
#pragma unroll
            for (int k = 0; k < 8; ++k) {
                v0[k] = xs[16 * tid + k];
                v1[k] = xs[16 * tid + 8 + k];
                m = fmaxf(m, fmaxf(fabsf(v0[k]), fabsf(v1[k])));
                sum += v0[k] + v1[k];
            }
            uint32_t w0[4][2], w1[4][2];
            digit_words(v0, m, w0);
            digit_words(v1, m, w1);
#pragma unroll
            for (int t = 0; t < 4; ++t)
                reinterpret_cast<uint4*>(dig)[tid * 4 + t] = make_uint4(w0[t][0], w0[t][1], w1[t][0], w1[t][1]);
            const float sc = m > 0.0f ? ldexpf(1.0f, ilogbf(m) - 5) : 0.0f;
            tab[tid] = make_float4(ldexpf(sc, -14), ldexpf(sc, -21), -32.0f * sum, 0.0f);
        }
        __syncthreads();  // the image is complete, and xs free for the next vector
    }

    const uint32_t g = lane >> 4, r = lane & 15;
    const bool aon = (r >> 2) == g;
    const uint32_t am = aon ? 256u : 0u;
    uint32_t a0[NV], t0[NV];
#pragma unroll
    for (int v = 0; v < NV; ++v) {
        const uint8_t* dig = img0 + (size_t)v * 5 * K;
        a0[v] = aon ? lds_addr(dig) + r * 16 : lds_addr(zero_blk);
        t0[v] = lds_addr(dig + (size_t)K * 4) + g * 16;
    }
    float bv[NV], acc[NV];
    uint32_t bi[NV], bad[NV];
#pragma unroll
    for (int v = 0; v < NV; ++v) {
        bv[v] = -INFINITY;
        acc[v] = 0.0f;
        bi[v] = 0xFFFFFFFFu;
        bad[v] = 0;
    }
    uint32_t ct = gw, cs = 0;
    auto record = [&](int u) {
        float sbacc[NV];
#pragma unroll
        for (int v = 0; v < NV; ++v) sbacc[v] = 0.0f;
#pragma unroll
        for (int kb = 0; kb < 4; ++kb) {
            const uint32_t wl0 = hr.code[u][(3 * kb) / 4][(3 * kb) % 4];
            const uint32_t wl1 = hr.code[u][(3 * kb + 1) / 4][(3 * kb + 1) % 4];
            const uint32_t wh = hr.code[u][(3 * kb + 2) / 4][(3 * kb + 2) % 4];
            const v4i bq = q6_unpack(wl0, wl1, wh);
            const uint32_t blk = cs * 4 + kb;
            const float ssc = (float)(int8_t)(hr.sc[u] >> (8 * kb));
#pragma unroll
            for (int v = 0; v < NV; ++v) {
                const v4i av = lds_at<v4i>(a0[v] + blk * am);
                const v4i d = __builtin_amdgcn_mfma_i32_16x16x64_i8(av, bq, v4i{0, 0, 0, 0}, 0, 0, 0);
                const v4f tb = lds_at<v4f>(t0[v] + blk * 64);
                const int I = (d[0] << 14) + (d[1] << 7) + d[2];
                float in = fmaf((float)I, tb.x, tb.z);
                in = fmaf((float)d[3], tb.y, in);
                sbacc[v] = fmaf(ssc, in, sbacc[v]);
            }
        }
        const float dr = h2f((uint16_t)hr.d[u]);
#pragma unroll
        for (int v = 0; v < NV; ++v) acc[v] = fmaf(dr, sbacc[v], acc[v]);
        fill(u);
        if (++cs == sb) {
            const uint32_t row = ct * 16 + r;
#pragma unroll
            for (int v = 0; v < NV; ++v) {
                const float val = row_total(acc[v]);
                acc[v] = 0.0f;
                if (lane < 16 && row < rows) {
                    if (!isfinite(val)) bad[v] = 1;
                    else if (better(val, row, bv[v], bi[v])) {
                        bv[v] = val;
                        bi[v] = row;
                    }
                }
            }
            cs = 0;
            ct += nw;
        }
    };
    for (uint32_t i = total / kHeadRing; i; --i) {
#pragma unroll
        for (int u = 0; u < kHeadRing; ++u) record(u);
    }
    const uint32_t rem = total % kHeadRing;
#pragma unroll
    for (int u = 0; u < kHeadRing - 1; ++u)
        if ((uint32_t)u < rem) record(u);
    __builtin_amdgcn_s_waitcnt(0x0F70);  // the ring's last requests (past the end) before exit

    // per vector: wave, then workgroup, then grid (greatest value, smallest id on ties, any flag)
#pragma unroll
    for (int v = 0; v < NV; ++v) {
#pragma unroll
        for (int o = 1; o < 64; o <<= 1) {
            const float ov = __shfl_xor(bv[v], o);
            const uint32_t oi = __shfl_xor(bi[v], o);
            if (better(ov, oi, bv[v], bi[v])) {
                bv[v] = ov;
                bi[v] = oi;
            }
            bad[v] |= __shfl_xor(bad[v], o);
        }
        if (lane == 0) {
            wv[wave][v] = bv[v];
            wi[wave][v] = bi[v];
            wb[wave][v] = bad[v];
        }
    }
    __syncthreads();
    const __amdgpu_buffer_rsrc_t prs = __builtin_amdgcn_make_buffer_rsrc(a.partial, 0, 0x7FFFFFFF, 0x00020000);
    if (tid < (uint32_t)NV) {
        const uint32_t v = tid;
        float b = wv[0][v];
        uint32_t id = wi[0][v], flag = wb[0][v];
        for (uint32_t w = 1; w < blockDim.x / 64; ++w) {
            if (better(wv[w][v], wi[w][v], b, id)) {
                b = wv[w][v];
                id = wi[w][v];
            }
            flag |= wb[w][v];
        }
        __builtin_amdgcn_raw_buffer_store_b128(v4u{__float_as_uint(b), id, flag, 0u}, prs, (blockIdx.x * NV + v) * 16, 0,
                                               kPartSC1);
    }
    __builtin_amdgcn_s_waitcnt(kWaitVm0);
    __syncthreads();
    if (tid == 0) {
        const uint32_t ticket = __hip_atomic_fetch_add(a.counter, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        last = ticket == gridDim.x - 1;
    }
    __syncthreads();
    if (!last) return;
    // the last workgroup: wave v < NV merges vector v's partials over the grid
    if (wave < (uint32_t)NV) {
        const uint32_t v = wave;
        float b = -INFINITY;
        uint32_t id = 0xFFFFFFFFu, flag = 0;
        for (uint32_t blk = lane; blk < gridDim.x; blk += 64) {
            const v4u p = __builtin_amdgcn_raw_buffer_load_b128(prs, (blk * NV + v) * 16, 0, kPartSC1);
            const float pv = __uint_as_float(p.x);
            if (better(pv, p.y, b, id)) {
                b = pv;
                id = p.y;
            }
            flag |= p.z;
        }
#pragma unroll
        for (int o = 1; o < 64; o <<= 1) {
            const float ov = __shfl_xor(b, o);
            const uint32_t oi = __shfl_xor(id, o);
            if (better(ov, oi, b, id)) {
                b = ov;
                id = oi;
            }
            flag |= __shfl_xor(flag, o);
        }
        if (lane == 0) {
            a.result[2 * v] = id;
            a.result[2 * v + 1] = flag || id >= rows;
        }
    }
    if (tid == 0) __hip_atomic_store(a.counter, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

hipError_t launch_head_batch(const HeadArgs& a, uint32_t nv, uint32_t vstride, uint32_t grid, hipStream_t s) {
    if (nv == 0 || nv > kHeadBatchMax || !a.result) return hipErrorInvalidValue;
    const size_t K = (size_t)a.w.units * 64, lds = K * 4 + nv * (K * 4 + K);  // xs, then per vector planes + table
    switch (nv) {
        case 1: hipLaunchKernelGGL(q6_head_batch_kernel<1>, dim3(grid), dim3(512), lds, s, a, vstride); break;
        case 2: hipLaunchKernelGGL(q6_head_batch_kernel<2>, dim3(grid), dim3(512), lds, s, a, vstride); break;
        case 3: hipLaunchKernelGGL(q6_head_batch_kernel<3>, dim3(grid), dim3(512), lds, s, a, vstride); break;
        case 4: hipLaunchKernelGGL(q6_head_batch_kernel<4>, dim3(grid), dim3(512), lds, s, a, vstride); break;
        default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

// ---- GQA decode attention ---------------------------------------------------------------------
//
// A flat grid of D-thread blocks over (slot, chunk), slot = token * kv_heads * query groups + KV
// head * query groups + query group: block b takes chunk (b / 8) % C of slot ((b / 8) / C) * 8 + b % 8
// (C = cmax, or 1 in ATT_APPEND), so the blocks of one slot are a multiple of 8 apart and, with
// workgroups dispatched to the 8 XCDs in turn, share an XCD.  The token of a slot indexes the batch (positions position + z,
// rows z * in_stride of q/k/v and z * out_stride of out).  Modes: ATT_DECODE
// appends the new K/V and attends; ATT_APPEND only normalises, rotates and appends K/V (grid x 1);
// ATT_ATTEND attends with every position's K/V already in the cache.  Each block takes one chunk of the
// visible range [max(0, pos + 1 - window), pos] for one KV head and its GQ
// query heads.  Prologue: q-norm + NeoX RoPE of the query heads (double angle,
// double rotation, f32 result); the block whose chunk ends at pos also
// normalises and rotates the new key, optionally normalises the value, rounds
// both to fp16 and appends them at slot pos % ring.  Then scores (16 lanes per
// token), chunk softmax, and p-weighted values; chunk partials (acc, max, sum)
// are merged by the last block of the slot.  XL: the slots' blocks share an XCD (the launch checked the
// dispatch order), so the partials and the ticket stay in that XCD's L2; otherwise they go through the
// memory side, where every XCD's accesses meet.

// RP: the q / k / v rows come from split-K partials (AttnArgs::raw_parts), a separate instance so
// that the decode path's code is unchanged by it.
__device__ __forceinline__ uint4 as_u4(v4u v) { return make_uint4(v.x, v.y, v.z, v.w); }

// Maximum and sum over the positions of one attention score step, whose LK lanes each hold one
// position's value: the 32-lane halves (and, at 16 lanes per position, the rows) swapped in registers.
template <int LK>
__device__ __forceinline__ float positions_max(float v) {
    const auto h = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    v = fmaxf(__uint_as_float(h[0]), __uint_as_float(h[1]));
    if constexpr (LK == 16) {
        const auto q = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
        v = fmaxf(__uint_as_float(q[0]), __uint_as_float(q[1]));
    }
    return v;
}
template <int LK>
__device__ __forceinline__ float positions_sum(float v) {
    if constexpr (LK == 16) {
        return row_total(v);
    } else {
        const auto h = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
        return __uint_as_float(h[0]) + __uint_as_float(h[1]);
    }
}

template <int D, int G, bool RP = false, bool XL = false, bool SH = false>
__global__ __launch_bounds__(D) void attention_kernel(AttnArgs a) {
    static_assert(D == 256 || D == 512, "one thread per channel");
    constexpr int NH = G + 2;     // this block's query heads, then the new key and value
    constexpr int W = D / 64;     // waves
    constexpr int LK = D / 16;    // lanes per token in the score loop (16 channels each)
    constexpr int KPW = 64 / LK;  // tokens per wave in one score-loop step
    constexpr int LV = D / 8;     // lanes per token in the value loop (8 channels each)
    constexpr int VPW = 64 / LV;  // tokens per wave in one value-loop step
    // SH: at most kAttnShortChunks chunks of at most kAttnMinChunk positions (every row returned to
    // the registers costs the CU's load-return bandwidth, so the first batches fit such a chunk)
    constexpr int UK = SH ? kAttnMinChunk / W / KPW : 8;  // cached K rows in flight per score-loop lane group
    constexpr int UV = SH ? kAttnMinChunk / W / VPW : 8;  // cached V rows in flight per value-loop lane group
    constexpr uint32_t kWaveTokens = kAttnMaxChunkLen / W;  // a wave's share of a chunk, at most
    __shared__ float rawl[NH][D];
    __shared__ float qs[G][D];
    __shared__ float sc[SH ? 1 : W][G][SH ? 1 : kWaveTokens];  // each wave's scores, then probabilities
    __shared__ __align__(16) float wacc[W][G][D];     // each wave's p-weighted value sums
    __shared__ float wml[W][G][2];                    // each wave's maximum and sum
    __shared__ double dred[W][NH];
    __shared__ __align__(16) float cw[G][kAttnMaxChunks];
    __shared__ __align__(16) float sl[G][kAttnMaxChunks];
    __shared__ bool last;
    constexpr int kStPol = XL ? kPartSC0 : kPartSC1, kLdPol = XL ? kPartNT : kPartSC1;
    constexpr int kScope = XL ? __HIP_MEMORY_SCOPE_WORKGROUP : __HIP_MEMORY_SCOPE_AGENT;

    const uint32_t tid = threadIdx.x, lane = tid & 63, wave = wave_id();
    if (a.state && a.state[ST_STOP]) return;
    const uint32_t qgroups = a.group / G, per_token = a.kv_heads * qgroups;
    const uint32_t cgrid = a.mode == ATT_APPEND ? 1u : a.cmax;
    const uint32_t slot = (blockIdx.x / 8 / cgrid) * 8 + blockIdx.x % 8, c = blockIdx.x / 8 % cgrid;
    if (slot >= a.tokens * per_token) return;
    const uint32_t z = slot / per_token;
    const uint32_t pos = (a.state ? a.state[ST_POS] : a.position) + z;
    const float* q_raw = a.q_raw + (size_t)z * a.in_stride;
    const float* k_raw = a.k_raw + (size_t)z * a.in_stride;
    const float* v_raw = a.v_raw + (size_t)z * a.in_stride;
    float* out = a.out + (size_t)z * a.out_stride;
    const uint32_t nvis = a.window ? min(pos + 1, a.window) : pos + 1;
    const uint32_t start = pos + 1 - nvis;
    uint32_t chunks = min(a.cmax, (nvis + a.min_chunk - 1) / a.min_chunk);
    const uint32_t clen = (nvis + chunks - 1) / chunks;
    chunks = (nvis + clen - 1) / clen;
    // chunk c of query heads kvh * group + qg * G + [0, G)
    const uint32_t kvh = slot % per_token / qgroups, qg = slot % qgroups;
    const uint32_t qh0 = kvh * a.group + qg * G;
    if (a.mode == ATT_APPEND ? qg != 0 && !a.q_out : c >= chunks) return;
    const uint32_t t0 = start + c * clen, t1 = min(pos + 1, t0 + clen);
    const uint32_t n = t1 - t0;
    const uint32_t ring = a.ring;
    // this chunk holds the new token (its K and V computed here)
    const bool has_new = a.mode == ATT_APPEND || (a.mode == ATT_DECODE && t1 == pos + 1);
    const bool append = has_new && qg == 0;  // and this block stores them in the cache
    const int nh = has_new ? NH : G;
    // Wave w takes the chunk's positions t0 + W k + w, k < nk: scores, softmax and p-weighted values
    // of its own positions, with no block barrier in between; the waves' partials are then combined.
    const uint32_t nk = n > wave ? (n - wave + W - 1) / W : 0u;

    // The prologue's inputs are requested first (vector loads return in issue order), then the
    // first batches of cached K and V rows, which the prologue's arithmetic does not wait for: rows
    // past the wave's positions clamped to the chunk's last one (the new token's row is read from
    // LDS instead; its cache slot may be written meanwhile).
    float raw[NH];
    if constexpr (RP) {
        // the partial planes, eight at a time, each round's loads issued before its sums
        size_t ro[NH];
#pragma unroll
        for (int h = 0; h < G; ++h) ro[h] = (size_t)(qh0 + h) * D + tid;
        ro[G] = (size_t)(a.k_raw - a.q_raw) + (size_t)kvh * D + tid;
        ro[G + 1] = (size_t)(a.v_raw - a.q_raw) + (size_t)kvh * D + tid;
        const float* p = a.raw_part + (size_t)z * a.raw_prow;
        const size_t plane = (size_t)a.raw_tp * a.raw_prow;
#pragma unroll
        for (int h = 0; h < NH; ++h) raw[h] = 0.0f;
        for (uint32_t k0 = 0; k0 < a.raw_parts; k0 += 8) {
            float pv[8][NH];
#pragma unroll
            for (int k = 0; k < 8; ++k)
#pragma unroll
                for (int h = 0; h < NH; ++h)
                    pv[k][h] = k0 + k < a.raw_parts && h < nh ? p[(k0 + k) * plane + ro[h]] : 0.0f;
#pragma unroll
            for (int k = 0; k < 8; ++k)
#pragma unroll
                for (int h = 0; h < NH; ++h)
                    if (k0 + k < a.raw_parts) raw[h] = k0 + k == 0 ? pv[k][h] : raw[h] + pv[k][h];
        }
    } else {
        // every load unconditional (a load under a branch is waited for at the branch's end)
#pragma unroll
        for (int h = 0; h < G; ++h) raw[h] = q_raw[(size_t)(qh0 + h) * D + tid];
        const float kr = k_raw[(size_t)kvh * D + tid], vr = v_raw[(size_t)kvh * D + tid];
        raw[G] = has_new ? kr : 0.0f;
        raw[G + 1] = has_new ? vr : 0.0f;
    }
    // thread j < D / 2 normalises and rotates the channel pair (j, j + D / 2)
    const bool pair = tid < D / 2;
    const uint32_t jh = tid % (D / 2);
    const float qw0 = a.q_norm[jh], qw1 = a.q_norm[jh + D / 2];
    const float kw0 = a.k_norm[jh], kw1 = a.k_norm[jh + D / 2];
    const double ifreq = a.inv_freq[jh];
    __builtin_amdgcn_sched_barrier(0);
    // The KV head's cache rows through buffer resources: with no bytes in ATT_APPEND, where the
    // loads below return zeros without a memory access (loads under a branch would be waited for
    // at its end, before the prologue).
    const uint32_t head_bytes = a.mode == ATT_APPEND ? 0u : ring * (uint32_t)D * 2u;
    const __amdgpu_buffer_rsrc_t krs = __builtin_amdgcn_make_buffer_rsrc(a.kcache + (size_t)kvh * ring * D, 0, head_bytes, 0x00020000);
    const __amdgpu_buffer_rsrc_t vrs = __builtin_amdgcn_make_buffer_rsrc(a.vcache + (size_t)kvh * ring * D, 0, head_bytes, 0x00020000);
    const uint32_t g = lane / LK, j = lane % LK;  // score loop: token slot, 16-channel slice
    uint4 kb[UK][2];
    auto load_k = [&](uint32_t k0) {
#pragma unroll
        for (int u = 0; u < UK; ++u) {
            const uint32_t k = k0 + KPW * u + g;
            const uint32_t off = ((t0 + min(W * k + wave, n - 1)) % ring * D + 16 * j) * 2;
            kb[u][0] = as_u4(__builtin_amdgcn_raw_buffer_load_b128(krs, off, 0, 0));
            kb[u][1] = as_u4(__builtin_amdgcn_raw_buffer_load_b128(krs, off + 16, 0, 0));
        }
    };
    const uint32_t hv = lane / LV, dl = lane % LV;  // value loop: token slot, 8-channel slice
    uint4 vb[SH ? 1 : UV];
    auto load_v = [&](uint32_t k0) {
#pragma unroll
        for (int u = 0; u < UV; ++u) {
            const uint32_t k = k0 + VPW * u + hv;
            vb[u] = as_u4(__builtin_amdgcn_raw_buffer_load_b128(vrs, ((t0 + min(W * k + wave, n - 1)) % ring * D + 8 * dl) * 2, 0, 0));
        }
    };
    // SH: one of the wave's positions per value row (VC channels per lane), every position of the
    // wave at once; rows past the wave's positions read as zeros (their probabilities are zero)
    constexpr int VC = D / 64, NT = kAttnMinChunk / W;
    using VRow = std::conditional_t<VC == 4, uint2, uint4>;
    VRow vs[SH ? NT : 1];
    load_k(0);
    if constexpr (SH) {
#pragma unroll
        for (int k = 0; k < NT; ++k) {
            const uint32_t off = (uint32_t)k < nk ? (((t0 + W * k + wave) % ring) * D + VC * lane) * 2 : 0x80000000u;
            if constexpr (VC == 4) {
                const v2u w = __builtin_amdgcn_raw_buffer_load_b64(vrs, off, 0, 0);
                vs[k] = make_uint2(w.x, w.y);
            } else {
                vs[k] = as_u4(__builtin_amdgcn_raw_buffer_load_b128(vrs, off, 0, 0));
            }
        }
    } else {
        load_v(0);
    }
    __builtin_amdgcn_sched_barrier(0);

    // ---- prologue: RMSNorm of the query heads (and the new K, V), then RoPE; two barriers
    double sn = 0.0, cs = 1.0;
    if (pair) sincos((double)pos * ifreq, &sn, &cs);
#pragma unroll
    for (int h = 0; h < NH; ++h) {
        const double v = wave_sum((double)raw[h] * (double)raw[h]);
        if (lane == 0) dred[wave][h] = v;
        rawl[h][tid] = raw[h];
    }
    __syncthreads();
    auto block_ss = [&](int h) {  // waves summed pairwise in index order
        if constexpr (W == 4) {
            return (dred[0][h] + dred[1][h]) + (dred[2][h] + dred[3][h]);
        } else {
            return ((dred[0][h] + dred[1][h]) + (dred[2][h] + dred[3][h])) +
                   ((dred[4][h] + dred[5][h]) + (dred[6][h] + dred[7][h]));
        }
    };
    // the new token's K (rotated) and V, fp16, for this block's reads: in the cache when this block
    // appends them, otherwise in LDS (another block of the KV head appends the same values)
    __shared__ uint16_t knew[D], vnew[D];
    if (pair) {
#pragma unroll
        for (int h = 0; h < G + 1; ++h) {
            if (h == G && !has_new) break;
            const double r = inv_rms_fast(block_ss(h), D, h < G ? a.q_eps : a.k_eps);
            const double x = (double)norm_apply(raw[h], r, h < G ? qw0 : kw0);
            const double y = (double)norm_apply(rawl[h][tid + D / 2], r, h < G ? qw1 : kw1);
            const float r0 = (float)__dsub_rn(__dmul_rn(x, cs), __dmul_rn(y, sn));
            const float r1 = (float)__dadd_rn(__dmul_rn(x, sn), __dmul_rn(y, cs));
            if (h < G) {
                qs[h][tid] = r0;
                qs[h][tid + D / 2] = r1;
            } else {
                knew[tid] = f2h(r0);
                knew[tid + D / 2] = f2h(r1);
            }
        }
    }
    if (has_new)
        vnew[tid] = f2h(a.v_norm ? (float)__dmul_rn((double)raw[G + 1], inv_rms_fast(block_ss(G + 1), D, a.v_eps)) : raw[G + 1]);
    __syncthreads();
    if (append) {
        const size_t slot_off = ((size_t)kvh * ring + pos % ring) * D;
        a.kcache[slot_off + tid] = knew[tid];
        a.vcache[slot_off + tid] = vnew[tid];
    }
    if (a.mode == ATT_APPEND) {
        if (a.q_out) {
#pragma unroll
            for (int gi = 0; gi < G; ++gi)
                a.q_out[((size_t)z * a.kv_heads * a.group + qh0 + gi) * D + tid] = qs[gi][tid];
        }
        return;
    }

    float mw[G], lw[G];
    if constexpr (SH) {
        // ---- scores of this wave's positions k = KPW u + g, u < UK (all of them), in registers:
        // the LK lanes of a position all hold its score (-inf past the wave's positions)
        float sd[UK][G];
        float qr[G][16];
#pragma unroll
        for (int gi = 0; gi < G; ++gi)
#pragma unroll
            for (int e = 0; e < 16; ++e) qr[gi][e] = qs[gi][16 * j + e];
#pragma unroll
        for (int u = 0; u < UK; ++u) {
            const uint32_t k = KPW * u + g, t = t0 + W * k + wave;
            uint4 k0v = kb[u][0], k1v = kb[u][1];
            if (has_new && t == pos) {
                k0v = *reinterpret_cast<const uint4*>(knew + 16 * j);
                k1v = *reinterpret_cast<const uint4*>(knew + 16 * j + 8);
            }
            const uint32_t kw[8] = {k0v.x, k0v.y, k0v.z, k0v.w, k1v.x, k1v.y, k1v.z, k1v.w};
            float kf[16];
#pragma unroll
            for (int e = 0; e < 8; ++e) {
                kf[2 * e] = h2f((uint16_t)(kw[e] & 0xFFFFu));
                kf[2 * e + 1] = h2f((uint16_t)(kw[e] >> 16));
            }
#pragma unroll
            for (int gi = 0; gi < G; ++gi) {
                float d = 0.0f;
#pragma unroll
                for (int e = 0; e < 16; ++e) d = fmaf(qr[gi][e], kf[e], d);
                d = row_sum(d);
                if constexpr (LK == 32) d += __shfl_xor(d, 16);  // the position's second row of 16 lanes
                sd[u][gi] = k < nk ? d * a.scale : -INFINITY;
            }
        }
        // ---- softmax over the wave's positions: across the KPW positions of a step with lane swaps
        float pr[UK][G];
#pragma unroll
        for (int gi = 0; gi < G; ++gi) {
            float mx = sd[0][gi];
#pragma unroll
            for (int u = 1; u < UK; ++u) mx = fmaxf(mx, sd[u][gi]);
            mx = positions_max<LK>(mx);
            float sum = 0.0f;
#pragma unroll
            for (int u = 0; u < UK; ++u) {
                pr[u][gi] = sd[u][gi] > -INFINITY ? expf(sd[u][gi] - mx) : 0.0f;
                sum += pr[u][gi];
            }
            mw[gi] = mx;
            lw[gi] = positions_sum<LK>(sum);
        }
        // ---- p-weighted values: position k's probability from lane (k % KPW) LK of its step
        float acc[G][VC];
#pragma unroll
        for (int gi = 0; gi < G; ++gi)
#pragma unroll
            for (int e = 0; e < VC; ++e) acc[gi][e] = 0.0f;
#pragma unroll
        for (int k = 0; k < NT; ++k) {
            if ((uint32_t)k >= nk) break;
            const uint32_t t = t0 + W * k + wave;
            VRow v = vs[k];  // (a conditional assignment, as for the K rows)
            if (has_new && t == pos) v = *reinterpret_cast<const VRow*>(vnew + VC * lane);
            uint32_t vw[VC / 2];
            if constexpr (VC == 4) {
                vw[0] = v.x;
                vw[1] = v.y;
            } else {
                vw[0] = v.x;
                vw[1] = v.y;
                vw[2] = v.z;
                vw[3] = v.w;
            }
            float vf[VC];
#pragma unroll
            for (int e = 0; e < VC / 2; ++e) {
                vf[2 * e] = h2f((uint16_t)(vw[e] & 0xFFFFu));
                vf[2 * e + 1] = h2f((uint16_t)(vw[e] >> 16));
            }
#pragma unroll
            for (int gi = 0; gi < G; ++gi) {
                const float pk = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(pr[k / KPW][gi]), (k % KPW) * LK));
#pragma unroll
                for (int e = 0; e < VC; ++e) acc[gi][e] = fmaf(pk, vf[e], acc[gi][e]);
            }
        }
#pragma unroll
        for (int gi = 0; gi < G; ++gi)
#pragma unroll
            for (int e = 0; e < VC; e += 4)
                *reinterpret_cast<float4*>(&wacc[wave][gi][VC * lane + e]) =
                    make_float4(acc[gi][e], acc[gi][e + 1], acc[gi][e + 2], acc[gi][e + 3]);
        if (lane == 0) {
#pragma unroll
            for (int gi = 0; gi < G; ++gi) {
                wml[wave][gi][0] = mw[gi];
                wml[wave][gi][1] = lw[gi];
            }
        }
    } else {
    // ---- scores of this wave's positions: LK lanes per position (16 channels each), KPW positions
    // per step, UK steps in flight
    float* const ws = &sc[wave][0][0];  // [G][kWaveTokens]
    {
        float qr[G][16];
#pragma unroll
        for (int gi = 0; gi < G; ++gi)
#pragma unroll
            for (int e = 0; e < 16; ++e) qr[gi][e] = qs[gi][16 * j + e];
        for (uint32_t k0 = 0; k0 < nk; k0 += UK * KPW) {
            if (k0) load_k(k0);
#pragma unroll
            for (int u = 0; u < UK; ++u) {
                const uint32_t k = k0 + KPW * u + g;
                if (k >= nk) break;
                const uint32_t t = t0 + W * k + wave;
                uint4 k0v = kb[u][0], k1v = kb[u][1];
                if (has_new && t == pos) {
                    k0v = *reinterpret_cast<const uint4*>(knew + 16 * j);
                    k1v = *reinterpret_cast<const uint4*>(knew + 16 * j + 8);
                }
                const uint32_t kw[8] = {k0v.x, k0v.y, k0v.z, k0v.w, k1v.x, k1v.y, k1v.z, k1v.w};
                float kf[16];
#pragma unroll
                for (int e = 0; e < 8; ++e) {
                    kf[2 * e] = h2f((uint16_t)(kw[e] & 0xFFFFu));
                    kf[2 * e + 1] = h2f((uint16_t)(kw[e] >> 16));
                }
#pragma unroll
                for (int gi = 0; gi < G; ++gi) {
                    float d = 0.0f;
#pragma unroll
                    for (int e = 0; e < 16; ++e) d = fmaf(qr[gi][e], kf[e], d);
                    d = row_sum(d);
                    if constexpr (LK == 32) d += __shfl_xor(d, 16);  // the position's second row of 16 lanes
                    if (j == 0) ws[gi * kWaveTokens + k] = d * a.scale;
                }
            }
        }
    }
    // the wave reads what its own lanes wrote to LDS: in order, no block barrier
    __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
    __builtin_amdgcn_wave_barrier();

    // ---- this wave's softmax: maximum, exponentials, sum
#pragma unroll
    for (int gi = 0; gi < G; ++gi) {
        float mx = -INFINITY;
        for (uint32_t k = lane; k < nk; k += 64) mx = fmaxf(mx, ws[gi * kWaveTokens + k]);
        mx = wave_max(mx);
        float sum = 0.0f;
        for (uint32_t k = lane; k < nk; k += 64) {
            const float p = expf(ws[gi * kWaveTokens + k] - mx);
            ws[gi * kWaveTokens + k] = p;
            sum += p;
        }
        mw[gi] = mx;
        lw[gi] = wave_sum(sum);
    }
    __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
    __builtin_amdgcn_wave_barrier();

    // ---- this wave's p-weighted values: LV lanes per position (8 channels each), VPW positions per
    // step, UV steps in flight; the VPW slots of a lane's channels added at the end
    {
        float acc[G][8];
#pragma unroll
        for (int gi = 0; gi < G; ++gi)
#pragma unroll
            for (int e = 0; e < 8; ++e) acc[gi][e] = 0.0f;
        for (uint32_t k0 = 0; k0 < nk; k0 += UV * VPW) {
            if (k0) load_v(k0);
#pragma unroll
            for (int u = 0; u < UV; ++u) {
                const uint32_t k = k0 + VPW * u + hv;
                if (k >= nk) break;
                const uint32_t t = t0 + W * k + wave;
                // (a conditional assignment: a select between the two loads would become a load
                // from a selected address, which keeps vb in memory)
                uint4 v = vb[u];
                if (has_new && t == pos) v = *reinterpret_cast<const uint4*>(vnew + 8 * dl);
                const uint32_t vw[4] = {v.x, v.y, v.z, v.w};
                float vf[8];
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    vf[2 * e] = h2f((uint16_t)(vw[e] & 0xFFFFu));
                    vf[2 * e + 1] = h2f((uint16_t)(vw[e] >> 16));
                }
#pragma unroll
                for (int gi = 0; gi < G; ++gi) {
                    const float p = ws[gi * kWaveTokens + k];
#pragma unroll
                    for (int e = 0; e < 8; ++e) acc[gi][e] = fmaf(p, vf[e], acc[gi][e]);
                }
            }
        }
        if constexpr (VPW == 2) {  // lanes l and l + 32 hold the same channels: one total in both
#pragma unroll
            for (int gi = 0; gi < G; ++gi)
#pragma unroll
                for (int e = 0; e < 8; ++e) {
                    const auto h = __builtin_amdgcn_permlane32_swap(__float_as_uint(acc[gi][e]),
                                                                    __float_as_uint(acc[gi][e]), false, false);
                    acc[gi][e] = __uint_as_float(h[0]) + __uint_as_float(h[1]);
                }
        }
        if (hv == 0) {  // written whatever nk (zeros for a wave with no positions)
#pragma unroll
            for (int gi = 0; gi < G; ++gi) {
                *reinterpret_cast<float4*>(&wacc[wave][gi][8 * dl]) = make_float4(acc[gi][0], acc[gi][1], acc[gi][2], acc[gi][3]);
                *reinterpret_cast<float4*>(&wacc[wave][gi][8 * dl + 4]) = make_float4(acc[gi][4], acc[gi][5], acc[gi][6], acc[gi][7]);
            }
        }
        if (lane == 0) {
#pragma unroll
            for (int gi = 0; gi < G; ++gi) {
                wml[wave][gi][0] = mw[gi];
                wml[wave][gi][1] = lw[gi];
            }
        }
    }
    }  // SH
    __syncthreads();

    // ---- the chunk's partial (channel tid): waves weighted by exp(m_w - M), in wave order (a wave
    // with no positions has m_w = -inf, weight 0; wave 0 always has one)
    float o[G], m[G], l[G];
#pragma unroll
    for (int gi = 0; gi < G; ++gi) {
        float M = wml[0][gi][0];
#pragma unroll
        for (int w = 1; w < W; ++w) M = fmaxf(M, wml[w][gi][0]);
        float ot = 0.0f, lt = 0.0f;
#pragma unroll
        for (int w = 0; w < W; ++w) {
            const float e = expf(wml[w][gi][0] - M);
            ot = fmaf(e, wacc[w][gi][tid], ot);
            lt = fmaf(e, wml[w][gi][1], lt);
        }
        o[gi] = ot;
        m[gi] = M;
        l[gi] = lt;
    }
    if (chunks == 1) {
#pragma unroll
        for (int gi = 0; gi < G; ++gi) out[(size_t)(qh0 + gi) * D + tid] = o[gi] / l[gi];
        return;
    }

    // ---- split-K merge: the last block of the slot combines the chunk partials
    // (a query head's partial row: D sums, max, sum, padding to whole 16-byte pieces)
    constexpr uint32_t R = attn_part_row(D);
    const size_t stride = (size_t)G * R;
    // Without XL the blocks of a slot may run on different XCDs, whose L2s are not coherent with
    // each other: the partials are stored through to the memory side (sc1) and waited for, the
    // ticket is an agent-scope atomic, and the last block reads the partials from the memory side,
    // so no L2 write-back or invalidation (a device-scope fence) is needed.  With XL they share one
    // XCD's L2: stores into it, a ticket in it, loads that miss the CU's L1 and hit it.
    const __amdgpu_buffer_rsrc_t prs =
        __builtin_amdgcn_make_buffer_rsrc(a.part + (size_t)slot * a.cmax * stride, 0, 0x7FFFFFFF, 0x00020000);
    const uint32_t mine = c * (uint32_t)stride * 4;  // this chunk's byte offset
#pragma unroll
    for (int gi = 0; gi < G; ++gi) {
        __builtin_amdgcn_raw_buffer_store_b32(__float_as_uint(o[gi]), prs, mine + (gi * R + tid) * 4, 0, kStPol);
        if (tid == 0)
            __builtin_amdgcn_raw_buffer_store_b64(v2u{__float_as_uint(m[gi]), __float_as_uint(l[gi])}, prs,
                                                  mine + (gi * R + D) * 4, 0, kStPol);
    }
    __builtin_amdgcn_s_waitcnt(kWaitVm0);
    __syncthreads();
    if (tid == 0) {
        const uint32_t ticket = __hip_atomic_fetch_add(a.counters + slot, 1u, __ATOMIC_RELAXED, kScope);
        last = ticket == chunks - 1;
    }
    __syncthreads();
    if (!last) return;
    // One round of loads: chunk (tid / G)'s maximum and sum of query head tid % G, and the first MU
    // of this thread's weighted-sum pieces: 16-byte piece f of the G query heads' sums in every P-th
    // chunk (chunks ph, ph + P, ...).  The maxima and sums go through LDS (one barrier); every
    // thread then takes the maximum M of its head and the weights exp(m_c - M) of its own chunks,
    // and the P phases' sums are added in order (a second barrier).
    constexpr uint32_t NF = G * D / 4, P = D / NF, MU = SH ? kAttnShortChunks / P : 16;
    static_assert(G * kAttnMaxChunks <= D, "one thread per (query head, chunk) maximum");
    const uint32_t f = tid % NF, ph = tid / NF, fg = f / (D / 4), f4 = f % (D / 4);
    const uint32_t c4 = (chunks + 3) & ~3u;  // chunks rounded up to whole float4 reads
    const bool has_ml = tid < chunks * G;
    v2u ml{0u, 0u};
    if (has_ml)
        ml = __builtin_amdgcn_raw_buffer_load_b64(prs, ((tid / G) * (uint32_t)stride + (tid % G) * R + D) * 4, 0, kLdPol);
    float4 pv[MU];
    auto load_pieces = [&](uint32_t k0) {
#pragma unroll
        for (uint32_t u = 0; u < MU; ++u) {
            const uint32_t k = min(k0 + u * P, chunks - 1);
            const v4u w = __builtin_amdgcn_raw_buffer_load_b128(prs, (k * (uint32_t)stride + fg * R + 4 * f4) * 4, 0, kLdPol);
            pv[u] = make_float4(__uint_as_float(w.x), __uint_as_float(w.y), __uint_as_float(w.z), __uint_as_float(w.w));
        }
    };
    load_pieces(ph);
    __builtin_amdgcn_s_waitcnt(kWaitVm0);
    if (tid < c4 * G) {  // past the last chunk: maximum -inf, sum 0
        cw[tid % G][tid / G] = has_ml ? __uint_as_float(ml.x) : -INFINITY;
        sl[tid % G][tid / G] = has_ml ? __uint_as_float(ml.y) : 0.0f;
    }
    __syncthreads();
    float M = -INFINITY;
    if (has_ml) {
        const float4* m4 = reinterpret_cast<const float4*>(cw[tid % G]);
        for (uint32_t q = 0; q < c4 / 4; ++q) {
            const float4 v = m4[q];
            M = fmaxf(M, fmaxf(fmaxf(v.x, v.y), fmaxf(v.z, v.w)));
        }
    }
    __syncthreads();
    if (tid < c4 * G) cw[tid % G][tid / G] = has_ml ? expf(__uint_as_float(ml.x) - M) : 0.0f;
    __syncthreads();
    float4 acc4 = make_float4(0.f, 0.f, 0.f, 0.f);
    float lp = 0.0f;  // sum over this thread's chunks of w_c l_c
    for (uint32_t k0 = ph;;) {
#pragma unroll
        for (uint32_t u = 0; u < MU; ++u) {
            const uint32_t k = k0 + u * P;
            if (k < chunks) {
                const float w = cw[fg][k];
                acc4.x = fmaf(w, pv[u].x, acc4.x);
                acc4.y = fmaf(w, pv[u].y, acc4.y);
                acc4.z = fmaf(w, pv[u].z, acc4.z);
                acc4.w = fmaf(w, pv[u].w, acc4.w);
                lp = fmaf(w, sl[fg][k], lp);
            }
        }
        k0 += MU * P;
        if (k0 >= chunks) break;
        load_pieces(k0);
    }
    static_assert(P * NF * 16 <= sizeof(wacc) && P * G == 4, "merge reduction layout");
    float4* red4 = reinterpret_cast<float4*>(&wacc[0][0][0]);  // [P][NF]
    __shared__ float redl[4];                                   // [P][G]: the sums of w_c l_c
    red4[ph * NF + f] = acc4;
    if (f4 == 0) redl[ph * G + fg] = lp;
    __syncthreads();
    if (tid < NF) {
        float4 t = red4[f];
        float il = redl[fg];
        for (uint32_t q = 1; q < P; ++q) {
            const float4 r = red4[q * NF + f];
            t.x += r.x;
            t.y += r.y;
            t.z += r.z;
            t.w += r.w;
            il += redl[q * G + fg];
        }
        float4 y;
        y.x = t.x / il;
        y.y = t.y / il;
        y.z = t.z / il;
        y.w = t.w / il;
        *reinterpret_cast<float4*>(out + (size_t)(qh0 + fg) * D + 4 * f4) = y;
    }
    if (tid == 0) __hip_atomic_store(a.counters + slot, 0u, __ATOMIC_RELAXED, kScope);
}

// Query heads per attention block: all of a KV head's at width 256 (1, 2 or 4), two at width 512
// (one for a single query head per KV head), so the block's LDS stays within bounds.
uint32_t attention_block_heads(uint32_t group, uint32_t head_width) {
    return head_width == 256 ? group : std::min<uint32_t>(group, 2u);
}

namespace {
template <int D, int G>
void launch_attention_dg(const AttnArgs& a, dim3 grid, hipStream_t s) {
    // the split-partial input only feeds the append pass (no merge); XL only changes the merge; SH
    // when the launch's position (known on the host) leaves at most kAttnShortChunks short chunks
    const bool sh = !a.state && a.mode != ATT_APPEND && a.cmax <= kAttnShortChunks && a.min_chunk == kAttnMinChunk &&
                    (a.window ? std::min(a.position + a.tokens, a.window) : a.position + a.tokens) <=
                        kAttnShortChunks * kAttnMinChunk;
    if (a.raw_parts) hipLaunchKernelGGL((attention_kernel<D, G, true>), grid, dim3(D), 0, s, a);
    else if (a.xcd_local && sh) hipLaunchKernelGGL((attention_kernel<D, G, false, true, true>), grid, dim3(D), 0, s, a);
    else if (a.xcd_local) hipLaunchKernelGGL((attention_kernel<D, G, false, true>), grid, dim3(D), 0, s, a);
    else if (sh) hipLaunchKernelGGL((attention_kernel<D, G, false, false, true>), grid, dim3(D), 0, s, a);
    else hipLaunchKernelGGL((attention_kernel<D, G>), grid, dim3(D), 0, s, a);
}
}  // namespace

hipError_t launch_attention(const AttnArgs& args, uint32_t group, uint32_t head_width, hipStream_t s, uint32_t tokens) {
    const uint32_t G = attention_block_heads(group, head_width);
    if (args.group != group || group % G || tokens == 0 || args.kv_heads == 0) return hipErrorInvalidValue;
    if (args.raw_parts && (args.mode != ATT_APPEND || !args.raw_part)) return hipErrorInvalidValue;
    AttnArgs a = args;
    a.tokens = tokens;
    // (slot, chunk) blocks, slots rounded up to whole groups of 8 (one per XCD)
    const uint64_t slots = (uint64_t)tokens * a.kv_heads * (group / G);
    const uint64_t blocks = (slots + 7) / 8 * 8 * (a.mode == ATT_APPEND ? 1u : a.cmax);
    if (blocks == 0 || blocks > 0x7FFFFFFFull) return hipErrorInvalidValue;
    const dim3 grid((uint32_t)blocks);
    if (head_width == 256) {
        switch (G) {
            case 1: launch_attention_dg<256, 1>(a, grid, s); break;
            case 2: launch_attention_dg<256, 2>(a, grid, s); break;
            case 4: launch_attention_dg<256, 4>(a, grid, s); break;
            default: return hipErrorInvalidValue;
        }
    } else if (head_width == 512) {
        switch (G) {
            case 1: launch_attention_dg<512, 1>(a, grid, s); break;
            case 2: launch_attention_dg<512, 2>(a, grid, s); break;
            default: return hipErrorInvalidValue;
        }
    } else {
        return hipErrorInvalidValue;
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

// Not after a step-kernel launch of this step timed out (ST_BAD 2): ST_POS then stays at the step's
// position, which the per-operation kernels run again.
__global__ void advance_kernel(uint32_t* state) {
    if (state[ST_BAD] != 2u) state[ST_POS] += 1u;
}

// Clears n words with vector stores (a kernel rather than a memset, so that a caller may capture
// it in a graph).
__global__ __launch_bounds__(256) void zero_words_kernel(uint32_t* p, uint32_t n) {
    for (uint32_t i = threadIdx.x; i < n; i += blockDim.x) p[i] = 0u;
}

hipError_t launch_zero_words(uint32_t* p, uint32_t n, hipStream_t s) {
    hipLaunchKernelGGL(zero_words_kernel, dim3(1), dim3(256), 0, s, p, n);
    return hipGetLastError();
}

// Final logit softcapping, crates/domain/src/q6.rs:66-71: y = tanh(x / cap) * cap, the quotient and
// product in f32 as the reference computes them and tanh in double rounded to f32.
__global__ __launch_bounds__(256) void softcap_kernel(const float* x, float* y, size_t n, float cap) {
    for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (size_t)gridDim.x * blockDim.x)
        y[i] = __fmul_rn((float)tanh((double)__fdiv_rn(x[i], cap)), cap);
}

hipError_t launch_softcap(const float* x, float* y, size_t n, float cap, hipStream_t s) {
    const size_t blocks = std::min<size_t>((n + 255) / 256, 4096);
    hipLaunchKernelGGL(softcap_kernel, dim3((uint32_t)blocks), dim3(256), 0, s, x, y, n, cap);
    return hipGetLastError();
}

hipError_t launch_advance(uint32_t* state, hipStream_t s) {
    hipLaunchKernelGGL(advance_kernel, dim3(1), dim3(1), 0, s, state);
    return hipGetLastError();
}

}  // namespace af
