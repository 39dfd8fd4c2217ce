// Fold-form measurement for gfx950: what folding one 1152-byte Q4_0 weight record (16 rows x 128
// columns: 1024 code bytes, 64 fp16 block scales) into fp32 row partials costs, with the records
// held in registers so that no memory traffic is involved, in two forms:
//   mfma - the decode kernels' form (device.h, step.hip:consume_one): the input as int8 digit
//          planes in LDS, two v_mfma_i32_16x16x64_i8 per record, then an integer and fp32 fold;
//   fma  - the plain form: the input as fp32 in LDS, one nibble-to-float conversion and one FMA
//          per weight, the block scale and the -8 offset once per block.
// Lane 16 q + r of a wave folds block q of row r of each record; the wave steps over super-tiles
// seven apart and writes a run's row sums at its end, as the step kernel's streaming waves do,
// seven such waves per workgroup beside an idle wave 0 (the step kernel's roles) on a grid of one
// workgroup per CU.  Prints each form's time per record and wave, the streaming rate that time
// caps a CU and the chip at, and checks that the two forms' row sums of one pass agree.
//
//   make -C adaforge_amd/csrc ../fold_forms && adaforge_amd/fold_forms
#include <cstdio>
#include <cstdlib>
#include <algorithm>
#include <cmath>
#include <vector>

#include "device.h"

namespace af {
namespace {

constexpr uint32_t kK = 3840, kNst = kK / 128, kRec = 8, kWaves = 8, kStreaming = 7;
constexpr uint32_t kPartRows = 4096;  // part[] floats (row sums, indexed as in the step kernel)
enum Form { F_MFMA = 0, F_FMA = 1 };

// LDS: [digit image kNst * 576][x fp32 kK][block sums kK / 32][part kPartRows][zero block 32]
constexpr uint32_t kImgOff = 0, kXOff = kNst * kStepImg, kSumOff = kXOff + 4 * kK, kPartOff = kSumOff + 4 * (kK / 32),
                   kZeroOff = kPartOff + 4 * kPartRows, kLds = kZeroOff + 32;

struct Cur {
    uint32_t st, prow;
};

// Wave w (1..7): super-tiles w - 1, w + 6, ... of a single row tile repeated; a run ends where the
// next step wraps past kNst, and its row sums go to part[prow + r] (prow advances by 128 per run,
// wrapping inside part).
__device__ __forceinline__ bool step_cur(Cur& c) {
    const uint32_t s1 = c.st + kStreaming;
    const bool wrap = s1 >= kNst;
    c.st = wrap ? s1 - kNst : s1;
    return wrap;
}

template <int F>
__device__ __forceinline__ void fold(const v4u code, uint32_t scale, uint32_t st, float& acc, const uint8_t* lds,
                                     uint32_t lane) {
    const uint32_t q = lane >> 4, r = lane & 15;
    if constexpr (F == F_MFMA) {
        const bool aon = (r >> 2) == q;
        const uint32_t pa = aon ? lds_addr(lds + kImgOff) + r * 32 + st * 512 : lds_addr(lds + kZeroOff);
        const v4f t = lds_at<v4f>(lds_addr(lds + kImgOff + kNst * 512) + (st * 4 + q) * 16);
        const BlockTab tb{t.x, t.y, t.z, t.w};
        const Q4Tile w{make_uint4(code.x, code.y, code.z, code.w), scale};
        q4_mfma_tile(w, lds_at<v4i>(pa), lds_at<v4i>(pa + 16), tb, acc);
    } else {
        const uint32_t xa = lds_addr(lds + kXOff) + (st * 128 + 32 * q) * 4;
        float x[32];
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const v4f t = lds_at<v4f>(xa + 16 * i);
            x[4 * i] = t.x, x[4 * i + 1] = t.y, x[4 * i + 2] = t.z, x[4 * i + 3] = t.w;
        }
        const float bsum = lds_at<float>(lds_addr(lds + kSumOff) + (st * 4 + q) * 4);
        constexpr uint32_t M = 0x0F0F0F0Fu;
        const uint32_t cw[4] = {code.x, code.y, code.z, code.w};
        float s = 0.0f;
#pragma unroll
        for (int k = 0; k < 4; ++k) {  // byte j: element j (low nibble) and j + 16 (high nibble)
            const uint32_t lo = cw[k] & M, hi = (cw[k] >> 4) & M;
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                s = fmaf((float)((lo >> (8 * e)) & 0xFFu), x[4 * k + e], s);
                s = fmaf((float)((hi >> (8 * e)) & 0xFFu), x[16 + 4 * k + e], s);
            }
        }
        acc = fmaf(h2f((uint16_t)scale), fmaf(-8.0f, bsum, s), acc);
    }
}

template <int F>
__global__ __launch_bounds__(512) void fold_forms_kernel(const float* x, const v4u* codes, const uint32_t* scales,
                                                         uint32_t rounds, float* out) {
    extern __shared__ __align__(16) uint8_t lds[];
    const uint32_t tid = threadIdx.x, lane = tid & 63, wave = wave_id();
    // the input's two images: one octet per thread (the four threads of a quad hold a block)
    if (tid < kK / 8) {
        float v[8];
#pragma unroll
        for (int e = 0; e < 8; ++e) v[e] = x[8 * tid + e];
        float m, sum;
        quad_stats(v, m, sum);
        const uint32_t b = tid >> 2, p = tid & 3;
        digits8(v, m, reinterpret_cast<int8_t*>(lds + kImgOff), b, p);
        if (p == 0) {
            reinterpret_cast<BlockTab*>(lds + kImgOff + kNst * 512)[b] = block_tab(m, sum);
            reinterpret_cast<float*>(lds + kSumOff)[b] = sum;
        }
#pragma unroll
        for (int e = 0; e < 8; ++e) reinterpret_cast<float*>(lds + kXOff)[8 * tid + e] = v[e];
    }
    for (uint32_t i = tid; i < kPartRows; i += blockDim.x) reinterpret_cast<float*>(lds + kPartOff)[i] = 0.0f;
    if (tid < 8) reinterpret_cast<uint32_t*>(lds + kZeroOff)[tid] = 0u;
    __syncthreads();
    if (wave != 0) {
        float* part = reinterpret_cast<float*>(lds + kPartOff);
        v4u code[kRec];
        uint32_t sc[kRec];
#pragma unroll
        for (uint32_t u = 0; u < kRec; ++u) {
            code[u] = codes[(wave * kRec + u) * 64 + lane];
            sc[u] = scales[(wave * kRec + u) * 64 + lane];
        }
        Cur c{wave - 1, wave * 16};
        float acc = 0.0f;
        for (uint32_t i = 0; i < rounds; ++i) {
#pragma unroll
            for (uint32_t u = 0; u < kRec; ++u) {
                code[u].x ^= i;  // a fresh record every round (the fold cannot be hoisted)
                const uint32_t st = c.st;
                fold<F>(code[u], sc[u], st, acc, lds, lane);
                if (step_cur(c)) {
                    part[c.prow + (lane & 15)] = row_total(acc);
                    acc = 0.0f;
                    c.prow = c.prow + 128 >= kPartRows ? wave * 16 : c.prow + 128;
                }
            }
        }
        part[c.prow + (lane & 15)] += row_total(acc);
    }
    __syncthreads();
    for (uint32_t i = tid; i < kPartRows; i += blockDim.x)
        out[blockIdx.x * kPartRows + i] = reinterpret_cast<const float*>(lds + kPartOff)[i];
}

void check(hipError_t e, const char* what) {
    if (e != hipSuccess) {
        fprintf(stderr, "fold_forms: %s: %s\n", what, hipGetErrorString(e));
        exit(1);
    }
}

uint32_t f2h_host(float f) { return __builtin_bit_cast(uint16_t, (_Float16)f); }

uint64_t lcg(uint64_t& s) {
    s = s * 6364136223846793005ull + 1442695040888963407ull;
    return s >> 33;
}

}  // namespace
}  // namespace af

int main() {
    using namespace af;
    int dev = 0, cus = 0;
    check(hipGetDevice(&dev), "hipGetDevice");
    check(hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev), "CU count");
    const uint32_t grid = (uint32_t)cus;
    uint64_t seed = 12345;
    std::vector<float> hx(kK);
    for (auto& v : hx) v = ((float)(lcg(seed) % 20001) - 10000.0f) * 1e-4f;
    const size_t nrec = (size_t)kWaves * kRec * 64;
    std::vector<uint32_t> hc(nrec * 4), hs(nrec);
    for (auto& v : hc) v = (uint32_t)lcg(seed);
    for (auto& v : hs) v = f2h_host(1e-3f * (float)(1 + lcg(seed) % 10));
    float *dx, *dout;
    v4u* dc;
    uint32_t* ds;
    check(hipMalloc(&dx, kK * 4), "hipMalloc");
    check(hipMalloc(&dc, nrec * 16), "hipMalloc");
    check(hipMalloc(&ds, nrec * 4), "hipMalloc");
    check(hipMalloc(&dout, (size_t)grid * kPartRows * 4 * 2), "hipMalloc");
    check(hipMemcpy(dx, hx.data(), kK * 4, hipMemcpyHostToDevice), "copy");
    check(hipMemcpy(dc, hc.data(), nrec * 16, hipMemcpyHostToDevice), "copy");
    check(hipMemcpy(ds, hs.data(), nrec * 4, hipMemcpyHostToDevice), "copy");

    // one pass (one round), both forms: the same row sums up to the input image's rounding
    fold_forms_kernel<F_MFMA><<<grid, 512, kLds>>>(dx, dc, ds, 1, dout);
    fold_forms_kernel<F_FMA><<<grid, 512, kLds>>>(dx, dc, ds, 1, dout + (size_t)grid * kPartRows);
    check(hipDeviceSynchronize(), "check pass");
    std::vector<float> o((size_t)grid * kPartRows * 2);
    check(hipMemcpy(o.data(), dout, o.size() * 4, hipMemcpyDeviceToHost), "copy back");
    double worst = 0.0, scale = 0.0;
    for (size_t i = 0; i < (size_t)grid * kPartRows; ++i) scale = std::max(scale, (double)std::fabs(o[i]));
    for (size_t i = 0; i < (size_t)grid * kPartRows; ++i)
        worst = std::max(worst, std::fabs((double)o[i] - (double)o[i + (size_t)grid * kPartRows]));
    const bool agree = scale > 0.0 && worst <= 1e-5 * scale;
    printf("check: max |mfma - fma| over the row sums = %.3g (largest |sum| %.3g): %s\n", worst, scale,
           agree ? "agree" : "DIFFER");

    const uint32_t rounds = 512;
    hipEvent_t e0, e1;
    check(hipEventCreate(&e0), "event");
    check(hipEventCreate(&e1), "event");
    printf("%-5s %12s %14s %16s %14s\n", "form", "us / launch", "ns / record", "GB/s per CU", "TB/s (chip)");
    for (int f = 0; f < 2; ++f) {
        std::vector<float> t;
        for (int rep = 0; rep < 7; ++rep) {
            check(hipEventRecord(e0), "record");
            if (f == F_MFMA) fold_forms_kernel<F_MFMA><<<grid, 512, kLds>>>(dx, dc, ds, rounds, dout);
            else fold_forms_kernel<F_FMA><<<grid, 512, kLds>>>(dx, dc, ds, rounds, dout);
            check(hipEventRecord(e1), "record");
            check(hipEventSynchronize(e1), "sync");
            float ms = 0.0f;
            check(hipEventElapsedTime(&ms, e0, e1), "elapsed");
            t.push_back(ms);
        }
        std::sort(t.begin(), t.end());
        const double us = 1e3 * t[t.size() / 2];
        const double ns_rec = 1e3 * us / (rounds * kRec);  // per record and wave
        const double cu_gbs = kStreaming * (double)kStepRecord / ns_rec;  // 7 streaming waves per CU
        printf("%-5s %12.1f %14.1f %16.1f %14.2f\n", f == F_MFMA ? "mfma" : "fma", us, ns_rec, cu_gbs,
               cu_gbs * grid / 1e3);
    }
    check(hipDeviceSynchronize(), "end");
    return agree ? 0 : 2;
}
