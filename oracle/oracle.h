/*
 * TEST INFRASTRUCTURE ONLY.  CPU restatement of AdaForge's FP64-accumulation
 * domain oracles (the crates/domain/src sources) and of the backend's CPU layer
 * chain (crates/cuda-backend/src/stack.rs:662-700).  Only tests/,
 * __graft_entry__.smoke() and bench.py's cpu_baseline leg may load it, and
 * only as the checker; the product library never links or calls it.
 *
 * Every function returns OR_OK (0) or OR_ERR (non-zero) for the inputs the
 * reference rejects (its Err(...) cases), writing nothing useful on error.
 * Row-parallel functions take a thread count; each row keeps the reference's
 * sequential summation order, so results are bit-identical for any count.
 *
 * Pinning status of each function (what independent check it meets) is
 * recorded in the header comment of oracle.c next to each definition.
 */
#ifndef ADAFORGE_ORACLE_H
#define ADAFORGE_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define OR_OK 0
#define OR_ERR 1

float or_half_to_f32(uint16_t bits);
uint16_t or_f32_to_half(float value);
float or_f16_round(float value);

int or_q4_validate(const uint8_t* bytes, size_t len, uint32_t columns, uint32_t rows);
int or_q4_matvec(const uint8_t* bytes, uint32_t columns, uint32_t rows, const float* x, double* y, int threads);

int or_q6_validate(const uint8_t* bytes, size_t len, uint32_t columns, uint32_t rows);
int or_q6_matvec(const uint8_t* bytes, uint32_t columns, uint32_t rows, const float* x, double* y, int threads);
int or_softcap(float value, float cap, float* out);

int or_rmsnorm_validate(const float* weights, uint32_t n, float eps);
int or_rmsnorm(const float* weights, uint32_t n, float eps, const float* x, size_t len, double* y);

int or_rope_validate(uint32_t width, double base, const float* factors, uint32_t context);
int or_rope(uint32_t width, double base, const float* factors, uint32_t context, const float* x, size_t len,
            uint32_t position, double* y);

/* window == 0 means no window (None). */
int or_attention_validate(uint32_t q_heads, uint32_t kv_heads, uint32_t width, uint32_t window, float scale);
int or_visible_range(uint32_t window, uint32_t tokens, uint32_t position, uint32_t* start, uint32_t* end);
int or_attention(uint32_t q_heads, uint32_t kv_heads, uint32_t width, uint32_t window, float scale, const float* q,
                 const float* keys, const float* values, uint32_t tokens, uint32_t position, double* out);
/* or_attention with the query heads split over `threads` threads (bit-identical results). */
int or_attention_mt(uint32_t q_heads, uint32_t kv_heads, uint32_t width, uint32_t window, float scale, const float* q,
                    const float* keys, const float* values, uint32_t tokens, uint32_t position, double* out,
                    int threads);

int or_attention_output(const uint8_t* o_bytes, uint32_t o_cols, uint32_t o_rows, const float* norm_w, float norm_eps,
                        const float* attention, const float* residual, double* out, int threads);

double or_gelu_tanh(double x);
/* post_w == NULL: no post-FFN norm (the FFN-block configuration); the tail is then f32(down) + x, times layer_scale. */
int or_ffn(const float* pre_w, float pre_eps, const uint8_t* gate, const uint8_t* up, const uint8_t* down,
           uint32_t hidden, uint32_t intermediate, const float* post_w, float post_eps, float layer_scale,
           const float* x, double* out, int threads);

int or_embedding(const uint8_t* table, uint32_t width, uint32_t vocabulary, const uint32_t* ids, size_t n, int scaled,
                 float* out);
int or_greedy(const float* logits, size_t n, uint32_t* id);

int or_compare(const double* reference, const float* actual, size_t n, double atol, double rtol, double* max_error,
               double* max_ratio, size_t* first_bad);

/* ---- whole-model chain ------------------------------------------------------------ */

typedef struct {
    const float* input_norm; float input_eps;
    const uint8_t* q; const uint8_t* k; const uint8_t* v; /* v may equal k: shared K/V weights */
    const float* q_norm; float q_eps;
    const float* k_norm; float k_eps;
    double rope_base; const float* rope_factors; uint32_t rope_context;
    uint32_t q_heads, kv_heads, head_width, window; float scale;
    const uint8_t* o; const float* post_attn_norm; float post_attn_eps;
    const float* ffn_norm; float ffn_eps;
    const uint8_t* gate; const uint8_t* up; const uint8_t* down;
    const float* post_ffn_norm; float post_ffn_eps; float layer_scale;
    int v_norm;      /* unit-weight RMSNorm on V (stack.rs:687-688) */
    int kv_fp16;     /* round K and V to fp16 at the cache boundary */
} or_layer;

/* One layer (stack.rs:670-700) on input x with a caller-owned K/V history; see oracle.c. */
int or_layer_forward(const or_layer* w, uint32_t hidden, uint32_t intermediate, const float* x, float* keys,
                     float* values, uint32_t position, int use_given_kv, float* k_new, float* v_new, float* y,
                     int threads);

typedef struct or_model or_model;

or_model* or_model_new(uint32_t hidden, uint32_t intermediate, uint32_t layers, const or_layer* layer_table,
                       const uint8_t* q6_table, uint32_t vocabulary, const float* final_norm, float final_eps,
                       uint32_t capacity, int threads);
void or_model_free(or_model* m);
void or_model_reset(or_model* m);
/* Consume one token at the next position; writes the last layer output (hidden floats)
 * and, if per_layer != NULL, every layer's output (layers * hidden floats). */
int or_model_step(or_model* m, uint32_t token, float* hidden_out, float* per_layer);
/* Final norm + Q6_K head on the last output: raw f64 logits (vocabulary). */
int or_model_logits(or_model* m, double* logits);
/* Greedy generation: prompt then max_new tokens, stopping on any stop id. */
int or_model_generate(or_model* m, const uint32_t* prompt, size_t n_prompt, const uint32_t* stop, size_t n_stop,
                      uint32_t max_new, uint32_t* ids_out, size_t* n_out, int* stopped, float* margins);

#ifdef __cplusplus
}
#endif
#endif
