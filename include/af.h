/*
 * af.h - C ABI of the MI355X (gfx950) batch-1 decode backend.
 *
 * Drop-in boundary for AdaForge's GPU adapter: a Rust FFI crate binds these
 * entry points to implement the application ports `GpuDiagnostics` and
 * `GenerationSession` (crates/application/src/lib.rs:28-187, 1092-1126) in
 * place of crates/cuda-backend (cudarc + NVRTC).  No HIP, CUDA or torch type
 * crosses it: host buffers are plain pointers and sizes, device buffers are
 * `void*`/typed pointers the caller obtained from HIP, streams are `void*`
 * (a hipStream_t; NULL = the null stream).
 *
 * Errors: every entry point returns AF_OK or an AF_ERR_* code and leaves a
 * message for af_last_error() (thread-local), mapping onto the reference's
 * DiagnosticError(String) (crates/application/src/lib.rs:17-25).  Invalid
 * arguments are rejected before any GPU work, as the reference validates
 * before any CUDA call (crates/cuda-backend/src/stack.rs:60-84).
 *
 * Threading: a handle is used by one thread at a time; sessions own one
 * private stream (crates/cuda-backend/src/stack.rs:863-866).
 *
 * Weight formats are GGUF's, as the reference's GGUF reader hands them over:
 * Q4_0 (18 bytes per 32 weights: fp16 d, 16 nibble bytes), Q6_K (210 bytes
 * per 256 weights), row-major [rows][blocks]; `columns` is the contiguous
 * dimension (crates/model-formats/src/gguf.rs, README.md:76).
 */
#ifndef ADAFORGE_AF_H
#define ADAFORGE_AF_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define AF_OK 0
#define AF_ERR_INVALID 1    /* rejected before any GPU work */
#define AF_ERR_DEVICE 2     /* HIP runtime or launch failure */
#define AF_ERR_NONFINITE 3  /* non-finite logits reached greedy selection */
#define AF_ERR_POISONED 4   /* the session failed earlier and must be closed */
#define AF_ERR_NO_DEVICE 5  /* no gfx950 device */

#define AF_MAX_CONTEXT 32768u  /* crates/cuda-backend/src/stack.rs:18 (MAX_CONTEXT) */
#define AF_MAX_NEW_TOKENS 128u /* crates/cuda-backend/src/stack.rs:1183 (1..=128 per generate) */
#define AF_MAX_PROMPT 32768u

/* Message of the last failure on this thread ("" if none). */
const char* af_last_error(void);

/* ---- device query: GpuDiagnostics::check (crates/application/src/lib.rs:178,
 *      crates/cuda-backend/src/lib.rs:208-300, device-identity part) ---------------------------- */
typedef struct {
    char name[256];
    char arch[64];             /* "gfx950..." */
    int32_t compute_units;
    uint64_t free_memory_bytes;
    uint64_t total_memory_bytes;
} af_device_info;
int af_device_query(af_device_info* out);

/* ---- host-level diagnostics ----------------------------------------------------------------- */

/* GPU half of GpuDiagnostics::check_matvec (crates/application/src/lib.rs:179-186 ->
 * crates/cuda-backend/src/matvec.rs:9-122).  Uploads the Q4_0 matrix (validated as
 * Q4Matrix::new, crates/domain/src/q4.rs:9-28), runs y = W x once for each of the
 * n_inputs vectors (inputs: [n_inputs][columns]), then 1 warm-up and
 * `timed_repetitions` timed launches on the last vector; outputs: [n_inputs][rows];
 * *median_ms: median kernel time (0 if timed_repetitions == 0).  The caller compares
 * against Q4Matrix::reference_matvec with compare() (matvec.rs:175-193). */
int af_matvec_run(const uint8_t* q4, size_t len, uint32_t columns, uint32_t rows, const float* inputs,
                  uint32_t n_inputs, uint32_t timed_repetitions, float* outputs, float* median_ms);

/* GPU half of GpuDiagnostics::check_rms_norm (crates/application/src/lib.rs:172-177 ->
 * crates/cuda-backend/src/rms_norm.rs:9-130): `vectors` rows of `width` normalised with
 * the weights (validated as RmsNorm::new, crates/domain/src/rms_norm.rs:8-16), 1 warm-up
 * and `timed_repetitions` timed launches; outputs: [vectors][width]. */
int af_rmsnorm_run(const float* weights, uint32_t width, float eps, const float* inputs, uint32_t vectors,
                   uint32_t timed_repetitions, float* outputs, float* median_ms);

/* ---- device-resident operators (device pointers, caller's stream) ---------------------------- */

typedef struct af_q4 af_q4; /* a Q4_0 matrix resident on the device */
typedef struct af_q6 af_q6; /* a Q6_K matrix resident on the device */

/* Q4Matrix upload (crates/domain/src/q4.rs:9-28 validation; crates/cuda-backend/src/matvec.rs:36-38). */
int af_q4_upload(const uint8_t* q4, size_t len, uint32_t columns, uint32_t rows, af_q4** out);
void af_q4_free(af_q4* m);
/* y[rows] = W x[columns] (kernels/ada/q4_matvec.cu q4_matvec, launched by matvec.rs:72-101). */
int af_q4_gemv(const af_q4* m, const float* x, float* y, void* stream);
/* y[t][rows] = W x[t][columns] for t < tokens, 1 <= tokens <= 32, with W read once for all
 * vectors (crates/cuda-backend/src/batch.rs:113-148 BatchKernels::matvec, MAX_BATCH = 32 at
 * batch.rs:10; kernels/ada/q4_batch.cu).  The vectors' digit image lives in library scratch shared by
 * all calls: calls that overlap on different streams race. */
int af_q4_gemm(const af_q4* m, const float* x, uint32_t tokens, float* y, void* stream);

/* Q6Matrix upload (crates/domain/src/q6.rs:8-20; crates/cuda-backend/src/logits.rs:292-316). */
int af_q6_upload(const uint8_t* q6, size_t len, uint32_t columns, uint32_t rows, af_q6** out);
void af_q6_free(af_q6* m);
/* Raw logits = W x and greedy selection (ResidentHead::project_gpu + GpuGreedy::select,
 * crates/cuda-backend/src/logits.rs:424-467, greedy.rs:135-184): result (device, 2 words)
 * receives [argmax id (largest value, smallest id on ties), non-finite flag]; logits
 * (device, rows floats) may be NULL. */
int af_q6_gemv_argmax(const af_q6* m, const float* x, float* logits, uint32_t* result, void* stream);

/* No counterpart in the reference: for callers that cannot allocate device memory (code under
 * HIP graph capture, tight serving loops, harnesses that forbid hipMalloc).  The same computation
 * and results as af_q6_gemv_argmax, but the kernel's scratch (a completion counter and one 16-byte
 * argmax partial per workgroup) lives in a fixed array inside the library, AF_NOALLOC_SCRATCH_BYTES
 * per GPU, held by each GPU the library runs on until the process ends, instead of memory the
 * library allocates on its first call.  It allocates nothing: no hipMalloc, no hipFree.  Every call
 * on one GPU shares that GPU's array, so calls that overlap on one GPU (on different streams, or
 * from different threads) race and must be serialised by the caller.  Matrices whose scratch would
 * exceed the array are rejected with AF_ERR_INVALID (the head runs at most 256 workgroups, so every
 * valid Q6_K matrix fits: 256 + 256 * 16 bytes). */
#define AF_NOALLOC_SCRATCH_BYTES 8192u
int af_q6_gemv_argmax_noalloc(const af_q6* m, const float* x, float* logits, uint32_t* result, void* stream);

/* RMSNorm of `vectors` contiguous rows (kernels/ada/rms_norm.cu rms_norm, rms_norm.rs:72-108). */
int af_rmsnorm(const float* x, const float* weights, float* y, uint32_t width, uint32_t vectors, float eps,
               void* stream);

/* Final logit softcapping y = tanh(x / cap) * cap over n device floats (crates/domain/src/q6.rs:66-71;
 * the GPU half of the capped logits ResidentHead / logits::check report, crates/cuda-backend/src/
 * logits.rs:70-201).  Greedy selection uses the raw logits (logits.rs:267-276). */
int af_softcap(const float* x, float* y, size_t n, float cap, void* stream);

/* Host-side weight descriptors, mirroring the domain types the ports borrow
 * (crates/application/src/lib.rs:919-927, 1049-1053). */
typedef struct {
    const float* weights; /* host, len floats */
    uint32_t len;
    float epsilon;
} af_rms_norm;

typedef struct {
    const uint8_t* bytes; /* host GGUF Q4_0 / Q6_K blocks */
    size_t len;
    uint32_t columns;
    uint32_t rows;
} af_matrix;

typedef struct {
    uint32_t width;       /* head width (pairs i, i + width/2) */
    double base;          /* theta */
    const float* factors; /* host, width/2 frequency divisors (crates/domain/src/rope.rs:11-34) */
    uint32_t context;
} af_rope_params;

typedef struct {
    uint32_t q_heads;
    uint32_t kv_heads;
    uint32_t width;
    uint32_t window; /* 0: global (None) */
    float scale;     /* score scale (crates/domain/src/attention.rs:11-35) */
} af_attention_config;

/* Ffn (crates/domain/src/ffn.rs:60-94): pre-norm, gate/up (tanh-GELU(gate) * up), down,
 * optional post-norm (post.weights NULL: none), then (post + x) * layer_scale. */
typedef struct {
    af_rms_norm pre;
    af_matrix gate, up, down;
    af_rms_norm post;
    float layer_scale;
} af_ffn_weights;

typedef struct af_ffn af_ffn;
int af_ffn_create(const af_ffn_weights* w, af_ffn** out);
void af_ffn_free(af_ffn* f);
/* FfnKernel::run (crates/cuda-backend/src/ffn.rs:290-516): y = Ffn(x); x, y device [hidden]. */
int af_ffn_run(af_ffn* f, const float* x, float* y, void* stream);

/* Decode attention for one token (AttentionKernel + prepare_qkv + cache append,
 * crates/cuda-backend/src/attention.rs:107-170, stack.rs:332-497): per-head RMSNorm and
 * NeoX RoPE of q and k at `position`, optional unit-weight RMSNorm of v, K/V rounded to
 * fp16 and appended at slot position % ring of the caches ([kv_heads][ring][width] fp16,
 * device), then softmax(scale q.k) v over [max(0, position + 1 - window), position].  Calls share
 * the library's split-K scratch: calls on different streams must not overlap.  A call whose RoPE
 * parameters differ from the previous call's waits for the device before it uploads them. */
typedef struct {
    const float* q;      /* device [q_heads][width], raw projection outputs */
    const float* k;      /* device [kv_heads][width] */
    const float* v;      /* device [kv_heads][width] */
    const float* q_norm; /* device [width] */
    const float* k_norm; /* device [width] */
    float q_eps, k_eps, v_eps;
    int32_t v_norm;
    af_rope_params rope; /* factors on the host */
    af_attention_config config;
    uint16_t* k_cache;   /* device fp16 */
    uint16_t* v_cache;
    uint32_t ring;       /* cache slots; >= window for local layers, >= position + 1 otherwise */
    uint32_t position;
    float* out;          /* device [q_heads][width] */
} af_attention_args;
int af_attention_decode(const af_attention_args* args, void* stream);

/* ---- generation session: GpuDiagnostics::open_session / generate and GenerationSession
 *      (crates/application/src/lib.rs:29-47, 1092-1126; crates/cuda-backend/src/stack.rs:820-966,
 *      1146-1480) -------------------------------------------------------------------------- */

#define AF_LAYER_V_NORM 1u /* unit-weight RMSNorm of V with the input-norm epsilon (stack.rs:687-688) */

typedef struct {
    af_rms_norm input_norm;
    af_matrix matrices[3];   /* q, k, v; v.bytes == k.bytes: V shares K's weights (stack.rs:172) */
    af_rms_norm head_norms[2];
    af_rope_params rope;
    af_attention_config attention;
    af_matrix output;        /* AttentionOutput (crates/domain/src/attention_output.rs) */
    af_rms_norm output_norm;
    af_ffn_weights ffn;
    uint32_t flags;
} af_layer_weights;

typedef struct {
    af_rms_norm norm;
    af_matrix matrix; /* tied Q6_K embedding / lm-head */
    float cap;        /* final softcap (selection uses raw logits, logits.rs:267-276) */
} af_output_head;

typedef struct {
    uint64_t prompt_tokens;
    uint64_t cached_tokens;
    double prefill_ms;
    double first_token_ms;
    int32_t has_first_token;
    uint64_t decode_tokens;
    double decode_ms;
    double total_ms;
} af_generation_stats; /* GenerationStats (crates/application/src/lib.rs:1067-1076) */

typedef void (*af_token_fn)(void* user, uint32_t id);
typedef struct af_session af_session;

/* open_session: uploads every layer and the head, allocates KV caches for `capacity`
 * tokens (1..AF_MAX_CONTEXT) and captures the decode step (one launch for every layer, then the
 * head with greedy selection) and the prefill step (the layers alone) as HIP graphs, replayed
 * once per token (crates/cuda-backend/src/stack.rs:1100-1145 captures its layers the same way).
 * Layers outside the persistent step kernel's limits (Gemma 4's 512-wide global layers) run on
 * the per-operation kernels, between one step-kernel launch per run of the other layers; such a
 * session launches its steps directly (no graph: the same rate, measured).  A model with no layer
 * the step kernel takes runs on the per-operation kernels alone, captured as graphs.  With
 * AF_DISABLE_GRAPHS set in the environment every session launches its steps directly. */
int af_session_open(const af_layer_weights* layers, uint32_t n_layers, const af_output_head* head,
                    uint32_t capacity, af_session** out);
/* GenerationSession::generate / generate_stream (stack.rs:1171-1386): prompt must extend the
 * session's cached tokens; at most max_new (1..AF_MAX_NEW_TOKENS) greedy ids, stopping before
 * any id in `stop` (non-empty).  on_token may be NULL.  ids_out holds >= max_new ids.
 * Environment switches read at af_session_open: AF_PREFILL_BATCH (prompt positions per batched
 * pass, default 32; 0 or 1: one decode step per position, as ADAFORGE_BATCH_PREFILL=0,
 * stack.rs:982-987); AF_SPECULATIVE=1 with AF_SPEC_DEPTH (default 11, at most 15): greedy
 * speculative decoding with prompt-lookup drafts verified in one batched pass (ADAFORGE_SPECULATIVE,
 * ADAFORGE_SPEC_DEPTH, stack.rs:1252-1338, 1485-1511).  A verification pass predicts each position
 * from the batched layers, which sum in another order than the decode step (the reference's batched
 * path is bit-identical to its own sequential one, stack.rs:1063-1064): the ids equal plain greedy
 * decoding's up to rounding, so they can differ where the top two logits of a step nearly tie. */
int af_session_generate(af_session* s, const uint32_t* prompt, size_t n_prompt, const uint32_t* stop,
                        size_t n_stop, uint32_t max_new, af_token_fn on_token, void* user, uint32_t* ids_out,
                        size_t* n_out, int32_t* stopped, af_generation_stats* stats);
/* GenerationSession::reset (stack.rs:1469-1480). */
int af_session_reset(af_session* s);
/* Speculative decoding counters since open: verification passes, draft tokens, accepted draft tokens
 * (the ADAFORGE_DIAGNOSTICS "SPECULATIVE" line, stack.rs:1332-1337). */
int af_session_speculation(const af_session* s, uint64_t* passes, uint64_t* drafted, uint64_t* accepted);
void af_session_close(af_session* s);

/* Per-kernel decode timing, the event-based ADAFORGE_TIMING_DECODE diagnostic
 * (crates/cuda-backend/src/stack.rs:1245-1251, 1340-1372) at kernel granularity: behaves as
 * af_session_generate without stop ids, but launches every step's kernels directly with a
 * hipEvent pair around each launch on the session stream.  The first max_new / 2 steps launch the
 * persistent step kernel plainly, the others with its in-kernel timeline on.  timings[] holds one
 * entry per kind: "layers" (plain launches of the step kernel), "layers_timeline" (the launches
 * that write the timeline) and "head" from the events; the step kernel's phases "qkv",
 * "attention", "o_proj", "gate_up", "down" and "barrier" from the timeline (one launch = one
 * layer); then "<phase>.<mark>" entries splitting the slowest workgroup's
 * phase at its marks and "<phase>.mean" (mean workgroup time).  bytes_per_launch is the
 * algorithmic HBM traffic (weights read) averaged over launches; n_timings <= capacity. */
typedef struct {
    char name[32];
    uint64_t launches;
    double total_ms;
    double bytes_per_launch;
} af_kernel_timing;
int af_session_profile(af_session* s, const uint32_t* prompt, size_t n_prompt, uint32_t max_new, uint32_t* ids_out,
                       size_t* n_out, af_kernel_timing* timings, size_t capacity, size_t* n_timings);

/* GpuDiagnostics::generate (crates/application/src/lib.rs:38-47, stack.rs:820-833): a session
 * sized prompt + max_new, one generation, closed. */
int af_generate(const af_layer_weights* layers, uint32_t n_layers, const af_output_head* head,
                const uint32_t* prompt, size_t n_prompt, const uint32_t* stop, size_t n_stop, uint32_t max_new,
                uint32_t* ids_out, size_t* n_out, int32_t* stopped, af_generation_stats* stats);

/* GPU half of GpuDiagnostics::check_layer_stack / check_logits (crates/application/src/lib.rs:49-66,
 * crates/cuda-backend/src/stack.rs:707-817): consumes `ids` at the session's next positions
 * with direct launches and returns every layer's output per token (layer_outputs:
 * [n][layers][hidden], may be NULL), the fp16 K and V each layer appended per token
 * (kv_appended: [n][layers][2][kv_rows] fp16 bits, kv_rows = the largest kv_heads * width, may be
 * NULL), the raw logits after the last token (logits: [vocabulary], may be NULL) and the final
 * RMSNorm input after the last token (hidden: [hidden], may be NULL).  The ids join the
 * session's cached tokens.  A token that a generation emitted last is cached but has not run
 * through the layers yet; it runs first, unreported. */
int af_session_trace(af_session* s, const uint32_t* ids, size_t n, float* layer_outputs, uint16_t* kv_appended,
                     float* logits, float* hidden);

/* ---- GGUF model files: GgufInspector (crates/model-formats/src/gguf.rs:10-540) and the Gemma 4
 *      layer assembly of crates/application/src/stack.rs:26-107 -------------------------------------- */
/* Tensor types (GGUF type ids; crates/domain/src/lib.rs:12-20 block layouts). */
#define AF_GGUF_F32 0u
#define AF_GGUF_F16 1u
#define AF_GGUF_Q4_0 2u
#define AF_GGUF_Q8_0 8u
#define AF_GGUF_Q6_K 14u
#define AF_GGUF_BF16 30u
/* Metadata value kinds (MetadataValue, crates/application/src/lib.rs): arrays of at most 4096
 * elements are kept (AF_GGUF_ARRAY), larger ones are summarised (AF_GGUF_ARRAY_SUMMARY). */
#define AF_GGUF_UNSIGNED 0
#define AF_GGUF_SIGNED 1
#define AF_GGUF_FLOAT 2
#define AF_GGUF_BOOL 3
#define AF_GGUF_TEXT 4
#define AF_GGUF_ARRAY 5
#define AF_GGUF_ARRAY_SUMMARY 6
#define AF_GGUF_WHOLE UINT64_MAX /* af_gguf_meta: the value itself rather than one array element */
typedef struct af_gguf af_gguf;  /* an indexed GGUF file, memory-mapped read-only */
typedef struct {
    uint32_t version;
    uint64_t tensors, metadata, data_offset, file_bytes;
} af_gguf_file;                   /* ModelInfo's header fields */
typedef struct {
    uint32_t type;                /* AF_GGUF_* tensor type */
    uint32_t n_dims;
    uint64_t dims[4];             /* contiguous dimension first (columns, rows) */
    uint64_t offset;              /* absolute file offset */
    uint64_t bytes;
} af_gguf_tensor_info;            /* TensorInfo (crates/domain/src/lib.rs) */
typedef struct {
    int32_t kind;                 /* AF_GGUF_UNSIGNED ... AF_GGUF_ARRAY_SUMMARY */
    uint64_t u;                   /* UNSIGNED; BOOL as 0 / 1 */
    int64_t i;                    /* SIGNED */
    double f;                     /* FLOAT */
    const char* text;             /* TEXT (owned by the af_gguf; not NUL-terminated when it holds NULs) */
    uint64_t length;              /* TEXT bytes, or ARRAY / ARRAY_SUMMARY elements */
    uint32_t element_type;        /* ARRAY / ARRAY_SUMMARY: GGUF type id of the elements */
} af_gguf_value;
/* GgufInspector::inspect (gguf.rs:419-540): reads and validates the header of a little-endian GGUF
 * v3 file (signature, version, at most 100000 tensors and keys, unique keys and tensor names,
 * general.alignment a power of two up to 1 MiB, known tensor types with whole blocks per row,
 * aligned offsets, every tensor inside the file, no overlaps, a 256 MiB header budget). */
int af_gguf_open(const char* path, af_gguf** out);
void af_gguf_close(af_gguf* g);
int af_gguf_info(const af_gguf* g, af_gguf_file* out);
/* Tensor `index` (file order) or tensor `name`. */
int af_gguf_tensor_at(const af_gguf* g, uint64_t index, const char** name, af_gguf_tensor_info* out);
int af_gguf_tensor(const af_gguf* g, const char* name, af_gguf_tensor_info* out);
/* len bytes of tensor `name` from byte `offset` (read_q4_matrix / read_q6_matrix / read_f32_vector /
 * read_rms_norm / read_embeddings take their bytes this way, gguf.rs:44-391). */
int af_gguf_read(const af_gguf* g, const char* name, uint64_t offset, void* dst, uint64_t len);
/* Metadata entry `index` (key order) or `key`; for a kept array, `element` selects one element
 * (AF_GGUF_WHOLE: the array itself). */
int af_gguf_meta_at(const af_gguf* g, uint64_t index, const char** key, af_gguf_value* out);
int af_gguf_meta(const af_gguf* g, const char* key, uint64_t element, af_gguf_value* out);
/* The generation session of a Gemma 4 file (load_generation + GpuDiagnostics::open_session,
 * crates/application/src/stack.rs:318-357, lib.rs:29-36): every block assembled as stack.rs:26-107
 * (V from K's weights when attn_v is absent, local layers' sliding window and RoPE base
 * freq_base_swa with unit factors, global layers' freq_base and rope_freqs factors, attention scale
 * 1.0, unit-weight V RMSNorm, optional layer_output_scale, the file's RMSNorm epsilon), the tied
 * Q6_K token_embd table as embedding and lm-head, final_logit_softcapping as the head's cap.  The
 * session owns device copies; the af_gguf may be closed afterwards. */
int af_gguf_session_open(const af_gguf* g, uint32_t capacity, af_session** out);

#ifdef __cplusplus
}
#endif
#endif
