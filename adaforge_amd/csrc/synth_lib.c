/*
 * Host-side generator library for the seeded synthetic workloads (tests and
 * bench).  Not part of the C-ABI boundary in include/af.h: the reference has
 * no counterpart (its fixtures are Rust test code), and nothing on the decode
 * path calls it.  Multi-threaded over blocks; output is independent of the
 * thread count because every block is a pure function of (seed, index).
 */
#include <pthread.h>
#include <stddef.h>
#include <stdint.h>

#include "synth.h"

uint64_t synth_tensor_seed(uint64_t base, const char* name) { return synth_seed(base, name); }

typedef struct {
    int kind; /* 0 q4, 1 q6, 2 normal, 3 q4 with signed scales */
    uint64_t seed;
    double a, b;
    uint8_t* out;
    float* fout;
    uint64_t begin, end;
} job;

static void* worker(void* p) {
    job* j = (job*)p;
    for (uint64_t i = j->begin; i < j->end; ++i) {
        if (j->kind == 0) synth_q4_block(j->seed, i, j->a, j->b, j->out + i * 18);
        else if (j->kind == 3) synth_q4_block_signed(j->seed, i, j->a, j->b, j->out + i * 18);
        else if (j->kind == 1) synth_q6_block(j->seed, i, j->a, j->b, j->out + i * 210);
        else j->fout[i] = synth_normal(j->seed, i, j->a, j->b);
    }
    return NULL;
}

static void run(int kind, uint64_t seed, double a, double b, uint8_t* out, float* fout, uint64_t n, int threads) {
    if (threads < 1) threads = 1;
    if (threads > 64) threads = 64;
    if ((uint64_t)threads > n) threads = n ? (int)n : 1;
    pthread_t tid[64];
    job jobs[64];
    uint64_t per = (n + (uint64_t)threads - 1) / (uint64_t)threads;
    int started = 0;
    for (int t = 0; t < threads; ++t) {
        uint64_t lo = (uint64_t)t * per, hi = lo + per > n ? n : lo + per;
        if (lo >= hi) break;
        jobs[t] = (job){kind, seed, a, b, out, fout, lo, hi};
        if (threads == 1 || pthread_create(&tid[started], NULL, worker, &jobs[t]) != 0) {
            worker(&jobs[t]);
            continue;
        }
        ++started;
    }
    for (int t = 0; t < started; ++t) pthread_join(tid[t], NULL);
}

/* rows x columns Q4_0 matrix in GGUF row-major block order (18 B per 32 weights). */
void synth_q4(uint64_t seed, uint32_t columns, uint32_t rows, double dlo, double dhi, uint8_t* out, int threads) {
    run(0, seed, dlo, dhi, out, NULL, (uint64_t)rows * (columns / 32), threads);
}

/* The same with |d| ~ U[dlo, dhi] and a random sign on d (synth_q4_block_signed). */
void synth_q4_signed(uint64_t seed, uint32_t columns, uint32_t rows, double dlo, double dhi, uint8_t* out,
                     int threads) {
    run(3, seed, dlo, dhi, out, NULL, (uint64_t)rows * (columns / 32), threads);
}

/* rows x columns Q6_K matrix in GGUF row-major super-block order (210 B per 256 weights). */
void synth_q6(uint64_t seed, uint32_t columns, uint32_t rows, double dlo, double dhi, uint8_t* out, int threads) {
    run(1, seed, dlo, dhi, out, NULL, (uint64_t)rows * (columns / 256), threads);
}

/* n floats mean + std * N(0,1). */
void synth_normal_vec(uint64_t seed, uint64_t n, double mean, double std, float* out, int threads) {
    run(2, seed, mean, std, NULL, out, n, threads);
}

uint16_t synth_half(float f) { return synth_f32_to_f16(f); }
