// HIP kernels for gfx950 (MI355X): the per-operation entry points of the decode step of a
// Q4_0 / Q6_K transformer (Q4_0 GEMV on the int8 matrix cores, Q6_K head with greedy argmax,
// GQA decode attention, RMSNorm).  Cross-workgroup results (attention chunks, argmax
// partials) are combined by the last workgroup to finish, found with a device-scope counter
// that the last workgroup resets, so the kernels can be replayed in a graph.
#include "device.h"

namespace af {

template <int T, int IN, int OUT, int Q>
__global__ __launch_bounds__(512) void q4_gemv_kernel(Q4Args a, uint32_t out_rows) {
    extern __shared__ __align__(16) uint8_t smem[];
    __shared__ double red[8];
    __shared__ float part[T][8][16];

    if (a.state && a.state[ST_STOP]) return;
    const uint32_t tid = threadIdx.x, lane = tid & 63, wave = wave_id();
    const uint32_t S = a.slices, tile = wave / S, sl = wave % S;
    const Q4View& m = (T == 2 && tile == 1) ? a.w2 : a.w;
    const uint32_t B = a.w.blocks, K = B * 32, nst = a.w.nst;
    const uint32_t per = (nst + S - 1) / S, st0 = min(nst, sl * per), st1 = min(nst, st0 + per);
    const uint32_t q = lane >> 4, n = lane & 15;  // D tile: rows 4q..4q+3, column n

    const uint4* codes = reinterpret_cast<const uint4*>(m.codes);
    const uint2* scales = reinterpret_cast<const uint2*>(m.scales);
    auto load = [&](Q4Tile (&buf)[kQ4Ahead], uint32_t c0) {
#pragma unroll
        for (int u = 0; u < kQ4Ahead; ++u) {
            const uint32_t st = c0 + u;
            if (st < st1) q4_tile_load(codes, scales, blockIdx.x, nst, st, lane, buf[u]);
        }
    };
    InputRegs<IN, Q> g;
    input_load<IN, Q>(a.in, K, nst, g);  // inputs first (see input_load)
    __builtin_amdgcn_sched_barrier(0);
    Q4Tile buf[kQ4Ahead];
    load(buf, st0);
    __builtin_amdgcn_sched_barrier(0);

    const size_t xs_bytes = IN == IN_EMBED ? (size_t)K * 4 : 0;
    int8_t* dig = reinterpret_cast<int8_t*>(smem + xs_bytes);
    DigitTab* tab = reinterpret_cast<DigitTab*>(smem + xs_bytes + (size_t)nst * 512);
    input_digits<IN, Q>(a.in, K, nst, g, reinterpret_cast<float*>(smem), dig, tab, red);
    __syncthreads();

    float acc[4] = {0.f, 0.f, 0.f, 0.f};
    for (uint32_t c0 = st0; c0 < st1; c0 += kQ4Ahead) {
#pragma unroll
        for (int u = 0; u < kQ4Ahead; ++u) {
            const uint32_t st = c0 + u;
            if (st >= st1) break;
            q4_mfma_tile(buf[u], st, dig, tab, lane, acc);
        }
        if (c0 + kQ4Ahead < st1) load(buf, c0 + kQ4Ahead);
    }
    // sum the 16 columns of each row, then the slices
    q4_row_sums(acc);
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

// Every GEMV block has 512 threads: T row tiles, each split over 8 / T waves by super-tile.
constexpr uint32_t kQ4Threads = 512;

template <int T, int IN, int OUT, int Q>
static hipError_t q4_launch3(Q4Args a, uint32_t out_rows, hipStream_t st) {
    const uint32_t tiles = (out_rows + 15) / 16;
    a.slices = kQ4Threads / 64 / T;
    const size_t lds = (IN == IN_EMBED ? (size_t)a.w.blocks * 32 * 4 : 0) + (size_t)a.w.nst * (512 + 128);
    hipLaunchKernelGGL((q4_gemv_kernel<T, IN, OUT, Q>), dim3(tiles), dim3(kQ4Threads), lds, st, a, out_rows);
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
    const int lane = threadIdx.x & 63, wave = (int)wave_id();
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

    const uint32_t tid = threadIdx.x, lane = tid & 63, wave = wave_id();
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
                    d = row_sum(d);
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
