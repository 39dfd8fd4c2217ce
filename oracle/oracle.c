/*
 * TEST INFRASTRUCTURE ONLY: CPU restatement of AdaForge's FP64-accumulation
 * oracles.  It is the checker for the HIP path, never part of it.
 *
 * Reference sources restated (paths under the AdaForge repository):
 *   crates/domain/src/q4.rs, q6.rs, rms_norm.rs, rope.rs, attention.rs,
 *   attention_output.rs, ffn.rs, embedding.rs, sampling.rs,
 *   crates/cuda-backend/src/matvec.rs:175-193 (compare),
 *   crates/cuda-backend/src/stack.rs:662-700 (layer chain, FP32 boundaries),
 *   crates/cuda-backend/src/logits.rs:180-190 (head: norm -> Q6_K raw logits).
 *
 * Arithmetic follows the reference operation by operation: f32 products where
 * Rust multiplies f32, f64 accumulation in the same loop order, one rounding
 * to f32 wherever the reference calls fp32()/`as f32`.  Build with
 * -ffp-contract=off so no multiply-add is fused.
 *
 * How each function is pinned (tests/test_oracle_*.py):
 *   or_half_to_f32   reference KATs (q4.rs:120-126) + all 65536 bit patterns
 *                    against numpy's float16 -> float32 conversion.
 *   or_f32_to_half   numpy float32 -> float16 (round-to-nearest-even) on all
 *                    fp16 neighbourhoods (every fp16 value, midpoints, +-1 ulp).
 *   or_q4_matvec     KAT q4.rs:89-106; validation KATs q4.rs:108-118; numpy
 *                    brute force (explicit dequantisation, float64 dot) on
 *                    random shapes; zero input; one-hot column extraction.
 *   or_q6_matvec     KAT q6.rs:203-214; all 64 codes x 16 signed sub-scales
 *                    (embedding.rs:83-111); numpy brute force from an
 *                    independent unpacker written from the GGUF layout.
 *   or_rmsnorm       KATs rms_norm.rs:46-73; closed form in numpy.
 *   or_rope          KATs rope.rs:157-190 (identity, 1-rad rotation, norm
 *                    preservation, suppressed pairs); complex-multiply form.
 *   or_attention     KATs attention.rs:116-142; numpy softmax closed form.
 *   or_attention_output / or_ffn   KATs attention_output.rs:42-56,
 *                    ffn.rs:159-177 (gelu values, zero branch) and numpy
 *                    composition of the pinned pieces.
 *   or_embedding     KAT embedding.rs:279-297 (all codes, signed scales).
 *   or_greedy        KAT sampling.rs:19-26 + numpy argmax (first index).
 *   or_compare       matvec.rs:198-205 cases + hand-computed ratios.
 *   or_model_*       composition of the above following stack.rs:670-700;
 *                    checked against a numpy re-composition of the pinned
 *                    pieces on a tiny model.
 */
#include "oracle.h"

#include <math.h>
#include <pthread.h>
#include <stdlib.h>
#include <string.h>

/* ---- fp16 ----------------------------------------------------------------------------- */

/* crates/domain/src/q4.rs:68-83 */
float or_half_to_f32(uint16_t bits) {
    float sign = (bits & 0x8000u) ? -1.0f : 1.0f;
    uint32_t exponent = (bits >> 10) & 31u;
    uint32_t mantissa = bits & 1023u;
    if (exponent == 0) return sign * (float)mantissa * 5.9604644775390625e-8f; /* 2^-24 */
    if (exponent == 31) return mantissa == 0 ? sign * INFINITY : NAN;
    uint32_t b = ((exponent + 112u) << 23) | (mantissa << 13);
    float v;
    memcpy(&v, &b, 4);
    return sign * v;
}

/* Round-to-nearest-even binary32 -> binary16: the fp16 KV-cache boundary. */
uint16_t or_f32_to_half(float f) {
    uint32_t x;
    memcpy(&x, &f, 4);
    uint32_t sign = (x >> 16) & 0x8000u;
    uint32_t a = x & 0x7FFFFFFFu;
    if (a >= 0x7F800000u) return (uint16_t)(sign | 0x7C00u | (a > 0x7F800000u ? 0x200u | ((a >> 13) & 0x3FFu) : 0u));
    if (a >= 0x477FF000u) return (uint16_t)(sign | 0x7C00u);
    if (a < 0x38800000u) {
        if (a < 0x33000000u) return (uint16_t)sign;
        uint32_t e = a >> 23, m = (a & 0x7FFFFFu) | 0x800000u, sh = 126u - e;
        uint32_t q = m >> sh, rem = m & ((1u << sh) - 1u), half = 1u << (sh - 1u);
        if (rem > half || (rem == half && (q & 1u))) q++;
        return (uint16_t)(sign | q);
    }
    uint32_t q = (((a >> 23) - 112u) << 10) | ((a & 0x7FFFFFu) >> 13);
    uint32_t rem = a & 0x1FFFu;
    if (rem > 0x1000u || (rem == 0x1000u && (q & 1u))) q++;
    return (uint16_t)(sign | q);
}

float or_f16_round(float v) { return or_half_to_f32(or_f32_to_half(v)); }

static int finite_f(float v) { return isfinite(v) != 0; }

/* ---- row-parallel driver ------------------------------------------------------------- */

typedef void (*row_fn)(const void* ctx, uint32_t row, double* out);
typedef struct {
    row_fn fn;
    const void* ctx;
    double* out;
    uint32_t begin, end;
} row_job;

static void* row_worker(void* p) {
    row_job* j = (row_job*)p;
    for (uint32_t r = j->begin; r < j->end; ++r) j->fn(j->ctx, r, &j->out[r]);
    return NULL;
}

static void run_rows(row_fn fn, const void* ctx, uint32_t rows, double* out, int threads) {
    if (threads < 1) threads = 1;
    if ((uint32_t)threads > rows) threads = (int)rows;
    if (threads <= 1) {
        for (uint32_t r = 0; r < rows; ++r) fn(ctx, r, &out[r]);
        return;
    }
    pthread_t tid[256];
    row_job jobs[256];
    if (threads > 256) threads = 256;
    uint32_t per = (rows + (uint32_t)threads - 1) / (uint32_t)threads;
    int n = 0;
    for (int t = 0; t < threads; ++t) {
        uint32_t b = (uint32_t)t * per, e = b + per > rows ? rows : b + per;
        if (b >= e) break;
        jobs[n] = (row_job){fn, ctx, out, b, e};
        if (pthread_create(&tid[n], NULL, row_worker, &jobs[n]) != 0) {
            row_worker(&jobs[n]); /* fall back to this thread: same order, same bits */
            continue;
        }
        ++n;
    }
    for (int t = 0; t < n; ++t) pthread_join(tid[t], NULL);
}

/* ---- Q4_0 ---------------------------------------------------------------------------- */

/* crates/domain/src/q4.rs:9-28 */
int or_q4_validate(const uint8_t* bytes, size_t len, uint32_t columns, uint32_t rows) {
    if (columns == 0 || rows == 0 || columns % 32 != 0) return OR_ERR;
    uint64_t size = (uint64_t)(columns / 32) * rows * 18u;
    if (size != (uint64_t)len) return OR_ERR;
    for (uint64_t b = 0; b < size; b += 18)
        if (!finite_f(or_half_to_f32((uint16_t)(bytes[b] | (bytes[b + 1] << 8))))) return OR_ERR;
    return OR_OK;
}

typedef struct {
    const uint8_t* bytes;
    uint32_t columns;
    const float* x;
} q4_ctx;

/* crates/domain/src/q4.rs:41-66, one row: FP32 weight, FP64 products and sum, block order. */
static void q4_row(const void* c, uint32_t row, double* out) {
    const q4_ctx* k = (const q4_ctx*)c;
    uint32_t blocks = k->columns / 32;
    const uint8_t* r = k->bytes + (size_t)row * blocks * 18;
    double sum = 0.0;
    for (uint32_t b = 0; b < blocks; ++b) {
        const uint8_t* blk = r + (size_t)b * 18;
        float scale = or_half_to_f32((uint16_t)(blk[0] | (blk[1] << 8)));
        const float* xb = k->x + (size_t)b * 32;
        for (int j = 0; j < 16; ++j) {
            int lo = (int)(blk[2 + j] & 15) - 8;
            int hi = (int)(blk[2 + j] >> 4) - 8;
            float wl = scale * (float)lo;
            float wh = scale * (float)hi;
            sum += (double)wl * (double)xb[j];
            sum += (double)wh * (double)xb[16 + j];
        }
    }
    *out = sum;
}

int or_q4_matvec(const uint8_t* bytes, uint32_t columns, uint32_t rows, const float* x, double* y, int threads) {
    if (columns == 0 || rows == 0 || columns % 32 != 0) return OR_ERR;
    for (uint32_t i = 0; i < columns; ++i)
        if (!finite_f(x[i])) return OR_ERR;
    q4_ctx c = {bytes, columns, x};
    run_rows(q4_row, &c, rows, y, threads);
    for (uint32_t r = 0; r < rows; ++r)
        if (!isfinite(y[r])) return OR_ERR;
    return OR_OK;
}

/* ---- Q6_K ---------------------------------------------------------------------------- */

/* crates/domain/src/q6.rs:8-20 */
int or_q6_validate(const uint8_t* bytes, size_t len, uint32_t columns, uint32_t rows) {
    if (columns == 0 || columns > 65536 || columns % 256 != 0 || rows == 0 || rows > 1000000) return OR_ERR;
    uint64_t size = (uint64_t)(columns / 256) * rows * 210u;
    if (size != (uint64_t)len) return OR_ERR;
    for (uint64_t b = 0; b < size; b += 210)
        if (!finite_f(or_half_to_f32((uint16_t)(bytes[b + 208] | (bytes[b + 209] << 8))))) return OR_ERR;
    return OR_OK;
}

typedef struct {
    const uint8_t* bytes;
    uint32_t columns;
    const float* x;
} q6_ctx;

/* crates/domain/src/q6.rs:36-65, one row: w = (d * f32(sc)) * f32(code - 32), f64 sum in
 * (super-block, group, quarter, lane) order. */
static void q6_row(const void* c, uint32_t row, double* out) {
    const q6_ctx* k = (const q6_ctx*)c;
    uint32_t blocks = k->columns / 256;
    const uint8_t* r = k->bytes + (size_t)row * blocks * 210;
    double sum = 0.0;
    for (uint32_t i = 0; i < blocks; ++i) {
        const uint8_t* b = r + (size_t)i * 210;
        float d = or_half_to_f32((uint16_t)(b[208] | (b[209] << 8)));
        const float* xb = k->x + (size_t)i * 256;
        for (int group = 0; group < 2; ++group)
            for (int quarter = 0; quarter < 4; ++quarter)
                for (int lane = 0; lane < 32; ++lane) {
                    uint8_t low = b[group * 64 + lane + (quarter % 2) * 32];
                    low = quarter < 2 ? (uint8_t)(low & 15) : (uint8_t)(low >> 4);
                    uint8_t high = (uint8_t)((b[128 + group * 32 + lane] >> (quarter * 2)) & 3);
                    int code = (int)(low | (high << 4)) - 32;
                    int8_t scale = (int8_t)b[192 + group * 8 + quarter * 2 + lane / 16];
                    float value = (d * (float)scale) * (float)code;
                    sum += (double)value * (double)xb[group * 128 + quarter * 32 + lane];
                }
    }
    *out = sum;
}

int or_q6_matvec(const uint8_t* bytes, uint32_t columns, uint32_t rows, const float* x, double* y, int threads) {
    if (columns == 0 || columns % 256 != 0 || rows == 0) return OR_ERR;
    for (uint32_t i = 0; i < columns; ++i)
        if (!finite_f(x[i])) return OR_ERR;
    q6_ctx c = {bytes, columns, x};
    run_rows(q6_row, &c, rows, y, threads);
    return OR_OK;
}

/* crates/domain/src/q6.rs:193-198 */
int or_softcap(float value, float cap, float* out) {
    if (!finite_f(value) || !finite_f(cap) || cap <= 0.0f) return OR_ERR;
    *out = tanhf(value / cap) * cap;
    return OR_OK;
}

/* ---- RMSNorm ------------------------------------------------------------------------- */

/* crates/domain/src/rms_norm.rs:8-16 */
int or_rmsnorm_validate(const float* w, uint32_t n, float eps) {
    if (n == 0 || n > 65536) return OR_ERR;
    for (uint32_t i = 0; i < n; ++i)
        if (!finite_f(w[i])) return OR_ERR;
    if (!finite_f(eps) || eps <= 0.0f) return OR_ERR;
    return OR_OK;
}

/* crates/domain/src/rms_norm.rs:24-41: direct weight multiply, FP64 throughout. */
int or_rmsnorm(const float* w, uint32_t n, float eps, const float* x, size_t len, double* y) {
    if (or_rmsnorm_validate(w, n, eps) != OR_OK) return OR_ERR;
    if (len == 0 || len % n != 0) return OR_ERR;
    for (size_t i = 0; i < len; ++i)
        if (!finite_f(x[i])) return OR_ERR;
    for (size_t base = 0; base < len; base += n) {
        double acc = 0.0;
        for (uint32_t i = 0; i < n; ++i) {
            double v = (double)x[base + i];
            acc += v * v;
        }
        double mean = acc / (double)n;
        double scale = 1.0 / sqrt(mean + (double)eps);
        for (uint32_t i = 0; i < n; ++i) y[base + i] = (double)x[base + i] * scale * (double)w[i];
    }
    return OR_OK;
}

/* ---- RoPE ---------------------------------------------------------------------------- */

/* crates/domain/src/rope.rs:11-34 */
int or_rope_validate(uint32_t width, double base, const float* factors, uint32_t context) {
    if (width == 0 || width > 65536 || width % 2 != 0 || !isfinite(base) || base <= 1.0 || context == 0) return OR_ERR;
    for (uint32_t i = 0; i < width / 2; ++i)
        if (!finite_f(factors[i]) || factors[i] <= 0.0f) return OR_ERR;
    return OR_OK;
}

/* crates/domain/src/rope.rs:52-77: NeoX pairs (i, i + width/2), FP64 angle and rotation. */
int or_rope(uint32_t width, double base, const float* factors, uint32_t context, const float* x, size_t len,
            uint32_t position, double* y) {
    if (or_rope_validate(width, base, factors, context) != OR_OK) return OR_ERR;
    if (len == 0 || len % width != 0 || position >= context) return OR_ERR;
    for (size_t i = 0; i < len; ++i)
        if (!finite_f(x[i])) return OR_ERR;
    uint32_t half = width / 2;
    for (size_t h = 0; h < len; h += width) {
        for (uint32_t i = 0; i < half; ++i) {
            double angle = (double)position * pow(base, -2.0 * (double)i / (double)width) / (double)factors[i];
            double s = sin(angle), c = cos(angle);
            double a = (double)x[h + i], b = (double)x[h + i + half];
            y[h + i] = a * c - b * s;
            y[h + i + half] = a * s + b * c;
        }
    }
    return OR_OK;
}

/* ---- attention ----------------------------------------------------------------------- */

/* crates/domain/src/attention.rs:11-35 (window 0 stands for None). */
int or_attention_validate(uint32_t q_heads, uint32_t kv_heads, uint32_t width, uint32_t window, float scale) {
    (void)window;
    if (q_heads == 0 || kv_heads == 0 || width == 0 || q_heads % kv_heads != 0) return OR_ERR;
    if (!finite_f(scale) || scale <= 0.0f) return OR_ERR;
    if ((uint64_t)q_heads * width > 0xFFFFFFFFull) return OR_ERR;
    return OR_OK;
}

/* crates/domain/src/attention.rs:52-65 */
int or_visible_range(uint32_t window, uint32_t tokens, uint32_t position, uint32_t* start, uint32_t* end) {
    if (tokens == 0 || position >= tokens) return OR_ERR;
    uint32_t e = position + 1;
    *end = e;
    *start = window ? (e > window ? e - window : 0) : 0;
    return OR_OK;
}

/* crates/domain/src/attention.rs:66-111: FP64 scores * scale, max-subtracted exp, normalise, sum p*v. */
/* One query head of or_attention (the loop body of attention.rs:66-111): scores in f64, the
 * max-subtracted exponentials, then sum_t p_t / denominator * v_t, in token order. */
typedef struct {
    uint32_t group, width;
    float scale;
    const float *q, *keys, *values;
    size_t start, n, stride;
    double* out;
} attn_job;

static void attention_head(const attn_job* a, uint32_t head, double* scores) {
    uint32_t kv = head / a->group;
    const float* query = a->q + (size_t)head * a->width;
    double max = -INFINITY;
    for (size_t t = 0; t < a->n; ++t) {
        const float* key = a->keys + (a->start + t) * a->stride + (size_t)kv * a->width;
        double s = 0.0;
        for (uint32_t c = 0; c < a->width; ++c) s += (double)query[c] * (double)key[c];
        s *= (double)a->scale;
        scores[t] = s;
        max = fmax(max, s);
    }
    double denominator = 0.0;
    for (size_t t = 0; t < a->n; ++t) {
        scores[t] = exp(scores[t] - max);
        denominator += scores[t];
    }
    double* o = a->out + (size_t)head * a->width;
    for (size_t t = 0; t < a->n; ++t) {
        const float* value = a->values + (a->start + t) * a->stride + (size_t)kv * a->width;
        double p = scores[t];
        for (uint32_t c = 0; c < a->width; ++c) o[c] += p / denominator * (double)value[c];
    }
}

typedef struct {
    const attn_job* a;
    uint32_t begin, end;
    int failed;
} attn_part;

static void* attention_worker(void* p) {
    attn_part* w = (attn_part*)p;
    double* scores = (double*)malloc((w->a->n ? w->a->n : 1) * sizeof(double));
    if (!scores) {
        w->failed = 1;
        return NULL;
    }
    for (uint32_t h = w->begin; h < w->end; ++h) attention_head(w->a, h, scores);
    free(scores);
    return NULL;
}

/* crates/domain/src/attention.rs:66-111.  With threads > 1 the query heads are split across
 * threads; each head runs the same loops, so the output is bit-identical to threads = 1. */
int or_attention_mt(uint32_t q_heads, uint32_t kv_heads, uint32_t width, uint32_t window, float scale, const float* q,
                    const float* keys, const float* values, uint32_t tokens, uint32_t position, double* out,
                    int threads) {
    if (or_attention_validate(q_heads, kv_heads, width, window, scale) != OR_OK) return OR_ERR;
    uint32_t start, end;
    if (or_visible_range(window, tokens, position, &start, &end) != OR_OK) return OR_ERR;
    size_t stride = (size_t)kv_heads * width;
    for (size_t i = 0; i < (size_t)q_heads * width; ++i)
        if (!finite_f(q[i])) return OR_ERR;
    for (size_t i = 0; i < (size_t)tokens * stride; ++i)
        if (!finite_f(keys[i]) || !finite_f(values[i])) return OR_ERR;
    memset(out, 0, sizeof(double) * (size_t)q_heads * width);
    attn_job a = {q_heads / kv_heads, width, scale, q, keys, values, start, end - start, stride, out};
    if (threads < 1) threads = 1;
    if ((uint32_t)threads > q_heads) threads = (int)q_heads;
    if (threads > 64) threads = 64;
    pthread_t tid[64];
    attn_part parts[64];
    uint32_t per = (q_heads + (uint32_t)threads - 1) / (uint32_t)threads;
    int n = 0, failed = 0;
    for (int t = 0; t < threads; ++t) {
        uint32_t b = (uint32_t)t * per, e = b + per > q_heads ? q_heads : b + per;
        if (b >= e) break;
        parts[t] = (attn_part){&a, b, e, 0};
        if (threads == 1 || pthread_create(&tid[n], NULL, attention_worker, &parts[t]) != 0) {
            attention_worker(&parts[t]); /* this thread: same order, same bits */
            continue;
        }
        ++n;
    }
    for (int t = 0; t < n; ++t) pthread_join(tid[t], NULL);
    for (int t = 0; t < threads && (uint32_t)t * per < q_heads; ++t) failed |= parts[t].failed;
    return failed ? OR_ERR : OR_OK;
}

int or_attention(uint32_t q_heads, uint32_t kv_heads, uint32_t width, uint32_t window, float scale, const float* q,
                 const float* keys, const float* values, uint32_t tokens, uint32_t position, double* out) {
    return or_attention_mt(q_heads, kv_heads, width, window, scale, q, keys, values, tokens, position, out, 1);
}

/* ---- output branch and FFN ----------------------------------------------------------- */

/* crates/domain/src/attention_output.rs:21-37: o-proj -> f32 -> RMSNorm -> f32 + residual. */
int or_attention_output(const uint8_t* o_bytes, uint32_t o_cols, uint32_t o_rows, const float* norm_w, float norm_eps,
                        const float* attention, const float* residual, double* out, int threads) {
    for (uint32_t i = 0; i < o_rows; ++i)
        if (!finite_f(residual[i])) return OR_ERR;
    double* proj = (double*)malloc(sizeof(double) * o_rows);
    float* proj32 = (float*)malloc(sizeof(float) * o_rows);
    int rc = OR_ERR;
    if (!proj || !proj32) goto done;
    if (or_q4_matvec(o_bytes, o_cols, o_rows, attention, proj, threads) != OR_OK) goto done;
    for (uint32_t i = 0; i < o_rows; ++i) proj32[i] = (float)proj[i];
    if (or_rmsnorm(norm_w, o_rows, norm_eps, proj32, o_rows, proj) != OR_OK) goto done;
    for (uint32_t i = 0; i < o_rows; ++i) out[i] = (double)(float)proj[i] + (double)residual[i];
    rc = OR_OK;
done:
    free(proj);
    free(proj32);
    return rc;
}

/* crates/domain/src/ffn.rs:95-97 */
double or_gelu_tanh(double x) {
    return 0.5 * x * (1.0 + tanh(sqrt(2.0 / 3.14159265358979323846) * (x + 0.044715 * x * x * x)));
}

/* crates/domain/src/ffn.rs:60-94 */
int or_ffn(const float* pre_w, float pre_eps, const uint8_t* gate, const uint8_t* up, const uint8_t* down,
           uint32_t hidden, uint32_t intermediate, const float* post_w, float post_eps, float layer_scale,
           const float* x, double* out, int threads) {
    int rc = OR_ERR;
    double* t64 = (double*)malloc(sizeof(double) * (hidden > intermediate ? hidden : intermediate));
    double* u64 = (double*)malloc(sizeof(double) * intermediate);
    float* normalized = (float*)malloc(sizeof(float) * hidden);
    float* active = (float*)malloc(sizeof(float) * intermediate);
    float* down32 = (float*)malloc(sizeof(float) * hidden);
    if (!t64 || !u64 || !normalized || !active || !down32) goto done;
    if (or_rmsnorm(pre_w, hidden, pre_eps, x, hidden, t64) != OR_OK) goto done;
    for (uint32_t i = 0; i < hidden; ++i) normalized[i] = (float)t64[i];
    if (or_q4_matvec(gate, hidden, intermediate, normalized, t64, threads) != OR_OK) goto done;
    if (or_q4_matvec(up, hidden, intermediate, normalized, u64, threads) != OR_OK) goto done;
    for (uint32_t i = 0; i < intermediate; ++i) {
        double g = (double)(float)t64[i];
        float gelu = (float)or_gelu_tanh(g);
        active[i] = gelu * (float)u64[i];
    }
    if (or_q4_matvec(down, intermediate, hidden, active, t64, threads) != OR_OK) goto done;
    for (uint32_t i = 0; i < hidden; ++i) down32[i] = (float)t64[i];
    if (post_w) {
        if (or_rmsnorm(post_w, hidden, post_eps, down32, hidden, t64) != OR_OK) goto done;
    } else {
        for (uint32_t i = 0; i < hidden; ++i) t64[i] = (double)down32[i];
    }
    for (uint32_t i = 0; i < hidden; ++i) out[i] = (double)((((float)t64[i]) + x[i]) * layer_scale);
    rc = OR_OK;
done:
    free(t64);
    free(u64);
    free(normalized);
    free(active);
    free(down32);
    return rc;
}

/* ---- embedding, greedy, compare ------------------------------------------------------ */

/* crates/domain/src/embedding.rs:8-33 (validation on the selected rows) and 53-78. */
int or_embedding(const uint8_t* table, uint32_t width, uint32_t vocabulary, const uint32_t* ids, size_t n, int scaled,
                 float* out) {
    if (width == 0 || width > 65536 || width % 256 != 0 || vocabulary == 0 || n == 0 || n > 256) return OR_ERR;
    size_t row_bytes = (size_t)(width / 256) * 210;
    for (size_t t = 0; t < n; ++t) {
        if (ids[t] >= vocabulary) return OR_ERR;
        const uint8_t* r = table + (size_t)ids[t] * row_bytes;
        for (size_t b = 0; b < row_bytes; b += 210)
            if (!finite_f(or_half_to_f32((uint16_t)(r[b + 208] | (r[b + 209] << 8))))) return OR_ERR;
    }
    float root = sqrtf((float)width);
    for (size_t t = 0; t < n; ++t) {
        const uint8_t* r = table + (size_t)ids[t] * row_bytes;
        for (uint32_t blk = 0; blk < width / 256; ++blk) {
            const uint8_t* b = r + (size_t)blk * 210;
            float d = or_half_to_f32((uint16_t)(b[208] | (b[209] << 8)));
            float* o = out + t * width + (size_t)blk * 256;
            for (int group = 0; group < 2; ++group)
                for (int lane = 0; lane < 32; ++lane)
                    for (int quarter = 0; quarter < 4; ++quarter) {
                        uint8_t low = b[group * 64 + lane + (quarter % 2) * 32];
                        low = quarter < 2 ? (uint8_t)(low & 15) : (uint8_t)(low >> 4);
                        uint8_t high = (uint8_t)((b[128 + group * 32 + lane] >> (quarter * 2)) & 3);
                        int quant = (int)(low | (high << 4)) - 32;
                        int8_t scale = (int8_t)b[192 + group * 8 + quarter * 2 + lane / 16];
                        float value = (d * (float)scale) * (float)quant;
                        o[group * 128 + quarter * 32 + lane] = scaled ? value * root : value;
                    }
        }
    }
    return OR_OK;
}

/* crates/domain/src/sampling.rs:2-16: strict maximum, smallest id on ties, non-finite rejected. */
int or_greedy(const float* logits, size_t n, uint32_t* id) {
    if (n == 0 || n > 0xFFFFFFFFull) return OR_ERR;
    for (size_t i = 0; i < n; ++i)
        if (!finite_f(logits[i])) return OR_ERR;
    size_t best = 0;
    for (size_t i = 1; i < n; ++i)
        if (logits[i] > logits[best]) best = i;
    *id = (uint32_t)best;
    return OR_OK;
}

/* crates/cuda-backend/src/matvec.rs:175-193 with (atol, rtol) as parameters. */
int or_compare(const double* reference, const float* actual, size_t n, double atol, double rtol, double* max_error,
               double* max_ratio, size_t* first_bad) {
    double me = 0.0, mr = 0.0;
    for (size_t i = 0; i < n; ++i) {
        double e = reference[i], v = (double)actual[i];
        double error = fabs(v - e);
        double ratio = error / (atol + rtol * fabs(e));
        if (!isfinite(e) || !isfinite(v) || ratio > 1.0) {
            if (first_bad) *first_bad = i;
            if (max_error) *max_error = error;
            if (max_ratio) *max_ratio = ratio;
            return OR_ERR;
        }
        if (error > me) me = error;
        if (ratio > mr) mr = ratio;
    }
    if (max_error) *max_error = me;
    if (max_ratio) *max_ratio = mr;
    return OR_OK;
}

/* ---- whole model: crates/cuda-backend/src/stack.rs:662-700 ---------------------------- */

struct or_model {
    uint32_t hidden, intermediate, layers, vocabulary, capacity;
    const or_layer* layer;
    const uint8_t* table;
    const float* final_norm;
    float final_eps;
    int threads;
    uint32_t position;
    float** keys;   /* per layer: capacity * kv_heads * width */
    float** values;
    float* x;       /* last output */
    float* ones;    /* unit weights for the V norm */
};

or_model* or_model_new(uint32_t hidden, uint32_t intermediate, uint32_t layers, const or_layer* layer_table,
                       const uint8_t* q6_table, uint32_t vocabulary, const float* final_norm, float final_eps,
                       uint32_t capacity, int threads) {
    or_model* m = (or_model*)calloc(1, sizeof(or_model));
    if (!m) return NULL;
    m->hidden = hidden;
    m->intermediate = intermediate;
    m->layers = layers;
    m->layer = layer_table;
    m->table = q6_table;
    m->vocabulary = vocabulary;
    m->final_norm = final_norm;
    m->final_eps = final_eps;
    m->capacity = capacity;
    m->threads = threads;
    m->keys = (float**)calloc(layers, sizeof(float*));
    m->values = (float**)calloc(layers, sizeof(float*));
    m->x = (float*)calloc(hidden, sizeof(float));
    uint32_t maxw = 1;
    for (uint32_t l = 0; l < layers; ++l) {
        const or_layer* w = &layer_table[l];
        size_t n = (size_t)capacity * w->kv_heads * w->head_width;
        m->keys[l] = (float*)malloc(n * sizeof(float));
        m->values[l] = (float*)malloc(n * sizeof(float));
        if (w->head_width > maxw) maxw = w->head_width;
    }
    m->ones = (float*)malloc(sizeof(float) * maxw);
    for (uint32_t i = 0; i < maxw; ++i) m->ones[i] = 1.0f;
    return m;
}

void or_model_free(or_model* m) {
    if (!m) return;
    for (uint32_t l = 0; l < m->layers; ++l) {
        free(m->keys[l]);
        free(m->values[l]);
    }
    free(m->keys);
    free(m->values);
    free(m->x);
    free(m->ones);
    free(m);
}

void or_model_reset(or_model* m) { m->position = 0; }

static void to_f32(const double* a, float* b, size_t n) {
    for (size_t i = 0; i < n; ++i) b[i] = (float)a[i];
}

/* One layer at `position` (crates/cuda-backend/src/stack.rs:670-700) on input x.  keys/values
 * hold (position + 1) * kv_rows floats; entries < position are the cache.  If use_given_kv,
 * entry `position` is taken as given; otherwise the layer's new K/V (normed, rotated, rounded
 * to fp16 when kv_fp16) are stored there.  k_new/v_new (may be NULL) receive the layer's own
 * new K/V before the fp16 rounding, either way, so a caller can compare a GPU's with them. */
int or_layer_forward(const or_layer* w, uint32_t hidden, uint32_t intermediate, const float* x, float* keys,
                     float* values, uint32_t position, int use_given_kv, float* k_new, float* v_new, float* y,
                     int threads) {
    uint32_t H = hidden, hw = w->head_width;
    uint32_t qn = w->q_heads * hw, kn = w->kv_heads * hw;
    uint32_t big = qn > H ? qn : H;
    double* t = (double*)malloc(sizeof(double) * (big > intermediate ? big : intermediate));
    float* normalized = (float*)malloc(sizeof(float) * H);
    float* q = (float*)malloc(sizeof(float) * qn);
    float* k = (float*)malloc(sizeof(float) * kn);
    float* v = (float*)malloc(sizeof(float) * kn);
    float* ones = (float*)malloc(sizeof(float) * hw);
    double* a64 = (double*)malloc(sizeof(double) * qn);
    float* a = (float*)malloc(sizeof(float) * qn);
    double* branch = (double*)malloc(sizeof(double) * H);
    float* branch32 = (float*)malloc(sizeof(float) * H);
    int rc = OR_ERR;
    if (!t || !normalized || !q || !k || !v || !ones || !a64 || !a || !branch || !branch32) goto done;
    for (uint32_t i = 0; i < hw; ++i) ones[i] = 1.0f;
    if (or_rmsnorm(w->input_norm, H, w->input_eps, x, H, t) != OR_OK) goto done;
    to_f32(t, normalized, H);
    if (or_q4_matvec(w->q, H, qn, normalized, t, threads) != OR_OK) goto done;
    to_f32(t, q, qn);
    if (or_q4_matvec(w->k, H, kn, normalized, t, threads) != OR_OK) goto done;
    to_f32(t, k, kn);
    if (or_q4_matvec(w->v, H, kn, normalized, t, threads) != OR_OK) goto done;
    to_f32(t, v, kn);
    if (or_rmsnorm(w->q_norm, hw, w->q_eps, q, qn, t) != OR_OK) goto done;
    to_f32(t, q, qn);
    if (or_rope(hw, w->rope_base, w->rope_factors, w->rope_context, q, qn, position, t) != OR_OK) goto done;
    to_f32(t, q, qn);
    if (or_rmsnorm(w->k_norm, hw, w->k_eps, k, kn, t) != OR_OK) goto done;
    to_f32(t, k, kn);
    if (or_rope(hw, w->rope_base, w->rope_factors, w->rope_context, k, kn, position, t) != OR_OK) goto done;
    to_f32(t, k, kn);
    if (w->v_norm) {
        if (or_rmsnorm(ones, hw, w->input_eps, v, kn, t) != OR_OK) goto done;
        to_f32(t, v, kn);
    }
    if (k_new) memcpy(k_new, k, sizeof(float) * kn); /* before the fp16 boundary */
    if (v_new) memcpy(v_new, v, sizeof(float) * kn);
    if (w->kv_fp16) {
        for (uint32_t i = 0; i < kn; ++i) {
            k[i] = or_f16_round(k[i]);
            v[i] = or_f16_round(v[i]);
        }
    }
    if (!use_given_kv) {
        memcpy(keys + (size_t)position * kn, k, sizeof(float) * kn);
        memcpy(values + (size_t)position * kn, v, sizeof(float) * kn);
    }
    if (or_attention(w->q_heads, w->kv_heads, hw, w->window, w->scale, q, keys, values, position + 1, position,
                     a64) != OR_OK)
        goto done;
    to_f32(a64, a, qn);
    if (or_attention_output(w->o, qn, H, w->post_attn_norm, w->post_attn_eps, a, x, branch, threads) != OR_OK)
        goto done;
    to_f32(branch, branch32, H);
    if (or_ffn(w->ffn_norm, w->ffn_eps, w->gate, w->up, w->down, H, intermediate, w->post_ffn_norm,
               w->post_ffn_eps, w->layer_scale, branch32, t, threads) != OR_OK)
        goto done;
    to_f32(t, y, H);
    rc = OR_OK;
done:
    free(t);
    free(normalized);
    free(q);
    free(k);
    free(v);
    free(ones);
    free(a64);
    free(a);
    free(branch);
    free(branch32);
    return rc;
}

static int layer_reference(or_model* m, uint32_t l, const float* x, float* y, uint32_t position) {
    if (position >= m->capacity) return OR_ERR;
    return or_layer_forward(&m->layer[l], m->hidden, m->intermediate, x, m->keys[l], m->values[l], position, 0, NULL,
                            NULL, y, m->threads);
}

int or_model_step(or_model* m, uint32_t token, float* hidden_out, float* per_layer) {
    if (m->position >= m->capacity) return OR_ERR;
    float* x = (float*)malloc(sizeof(float) * m->hidden);
    float* y = (float*)malloc(sizeof(float) * m->hidden);
    int rc = OR_ERR;
    if (!x || !y) goto done;
    if (or_embedding(m->table, m->hidden, m->vocabulary, &token, 1, 1, x) != OR_OK) goto done;
    for (uint32_t l = 0; l < m->layers; ++l) {
        if (layer_reference(m, l, x, y, m->position) != OR_OK) goto done;
        if (per_layer) memcpy(per_layer + (size_t)l * m->hidden, y, sizeof(float) * m->hidden);
        float* s = x;
        x = y;
        y = s;
    }
    memcpy(m->x, x, sizeof(float) * m->hidden);
    if (hidden_out) memcpy(hidden_out, x, sizeof(float) * m->hidden);
    m->position++;
    rc = OR_OK;
done:
    free(x);
    free(y);
    return rc;
}

/* crates/cuda-backend/src/logits.rs:180-190: f32(norm(x)) then Q6_K raw logits. */
int or_model_logits(or_model* m, double* logits) {
    double* n64 = (double*)malloc(sizeof(double) * m->hidden);
    float* n32 = (float*)malloc(sizeof(float) * m->hidden);
    int rc = OR_ERR;
    if (!n64 || !n32) goto done;
    if (or_rmsnorm(m->final_norm, m->hidden, m->final_eps, m->x, m->hidden, n64) != OR_OK) goto done;
    to_f32(n64, n32, m->hidden);
    rc = or_q6_matvec(m->table, m->hidden, m->vocabulary, n32, logits, m->threads);
done:
    free(n64);
    free(n32);
    return rc;
}

/* Greedy loop with the reference's order (stack.rs:1339-1363): select, stop check, consume. */
int or_model_generate(or_model* m, const uint32_t* prompt, size_t n_prompt, const uint32_t* stop, size_t n_stop,
                      uint32_t max_new, uint32_t* ids_out, size_t* n_out, int* stopped, float* margins) {
    double* logits = (double*)malloc(sizeof(double) * m->vocabulary);
    float* l32 = (float*)malloc(sizeof(float) * m->vocabulary);
    int rc = OR_ERR;
    *n_out = 0;
    *stopped = 0;
    if (!logits || !l32) goto done;
    for (size_t i = 0; i < n_prompt; ++i)
        if (or_model_step(m, prompt[i], NULL, NULL) != OR_OK) goto done;
    for (uint32_t s = 0; s < max_new; ++s) {
        if (or_model_logits(m, logits) != OR_OK) goto done;
        to_f32(logits, l32, m->vocabulary);
        uint32_t id;
        if (or_greedy(l32, m->vocabulary, &id) != OR_OK) goto done;
        if (margins) {
            float second = -INFINITY;
            for (uint32_t i = 0; i < m->vocabulary; ++i)
                if (i != id && l32[i] > second) second = l32[i];
            margins[s] = l32[id] - second;
        }
        int is_stop = 0;
        for (size_t j = 0; j < n_stop; ++j)
            if (stop[j] == id) is_stop = 1;
        if (is_stop) {
            *stopped = 1;
            break;
        }
        if (or_model_step(m, id, NULL, NULL) != OR_OK) goto done;
        ids_out[(*n_out)++] = id;
    }
    rc = OR_OK;
done:
    free(logits);
    free(l32);
    return rc;
}
