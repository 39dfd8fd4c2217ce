// Internal declarations shared by the HIP kernels (kernels.hip) and the host
// library (api.hip).  Nothing here crosses the C-ABI boundary in include/af.h.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <string>

namespace af {

// ---- device-resident weight layouts ----------------------------------------------------------
//
// Q4_0 (GGUF: 18 B per 32 weights) is retiled at upload for the matrix-core GEMV.
// Rows are grouped in tiles of 16 and blocks in super-tiles of 4 (128 columns), both
// zero-padded; each (row tile rt, super-tile st) owns one contiguous 1 KB code tile
// and one 128 B scale tile:
//   codes  [rt][st][4 blocks][16 rows][16]  the block's nibble bytes, unchanged
//                                           (byte j: low nibble = weight j, high = j + 16)
//   scales [rt][st][4 blocks][16 rows]      the block's fp16 d
// so one 16-byte load per lane, lane l at byte 16 l (block l / 16, row l % 16: the matrix
// cores' A-operand layout), reads a whole 16 x 128 tile with a wave in address order.
struct Q4View {
    const uint8_t* codes;
    const uint16_t* scales;
    uint32_t rows;    // real rows
    uint32_t blocks;  // real columns / 32
    uint32_t nst;     // super-tiles per row tile: ceil(blocks / 4)
};

// Q6_K (GGUF: 210 B per 256 weights) is split into "units" of 64 weights.  Unit
// u = 4 * superblock + 2 * g + hh (g: 128-element half, hh: 16-lane half of
// the 32-lane quarter) covers elements 128 g + 32 q + 16 hh + j for q in 0..3,
// j in 0..15, and stores:
//   a [rows][units][16]  ql[64 g + 16 hh + j]        (q = 0 low nibble, q = 2 high)
//   b [rows][units][16]  ql[64 g + 32 + 16 hh + j]   (q = 1 low nibble, q = 3 high)
//   h [rows][units][16]  qh[32 g + 16 hh + j]        (bits 2q, 2q+1 = high code bits)
//   s [rows][units]      4 int8 sub-scales sc[8 g + 2 q + hh], q = 0..3
//   d [rows][superblocks] fp16 super-scale
struct Q6View {
    const uint8_t* a;
    const uint8_t* b;
    const uint8_t* h;
    const uint32_t* s;
    const uint16_t* d;
    uint32_t rows;
    uint32_t units;  // columns / 64
    const uint8_t* t;  // head records: [ceil(rows / 16)][columns / 256][kQ6Rec] (upload_q6)
};

// A head record: 16 rows x one 256-weight super-block.  Lane l = 16 g + r (row r of the tile,
// 16-element group g of a 64-weight k-block kb) owns 12 code dwords (3 per kb: L0, L1, H) at
// [p = q / 4][l][q % 4] for dword q, its sub-block scales sc[r][4 kb + g] at 3072 + 4 l (byte kb),
// and the row's d at 3328 + 2 r.  L0 byte b = c_b | c_{4+b} << 4 (low nibbles), L1 byte b =
// c_{8+b} | c_{12+b} << 4, H byte b = the high bit pairs of c_b, c_{4+b}, c_{8+b}, c_{12+b}, where
// c_j is the 6-bit code of weight 64 kb + 16 g + j.
constexpr uint32_t kQ6Rec = 3360;

// ---- input stages (the GEMV prologue builds the fp32 input vector in LDS) -------------------
enum InputKind : int {
    IN_PLAIN = 0,  // x
    IN_NORM = 1,   // f32(rms(x) * w_n)
    IN_RESID = 2,  // v = (f32(rms(x) * w_a) + res) * scale  [w_a null: (x + res) * scale];
                   // block 0 stores v to x_out; input = f32(rms(v) * w_n)
    IN_EMBED = 3,  // v = Q6_K row ids[state[0]] * emb_scale; block 0 stores v; input = f32(rms(v) * w_n)
    IN_DIGITS = 4, // the input's digit image (below), written by the producing kernel
};

// Int8 digit form of an fp32 vector for the matrix-core GEMV: block b of 32 elements is
// s_b (q0 + q1 2^-7 + q2 2^-14 + q3 2^-21), s_b = 2^(ilogb(max |x|) - 5).  The image of a vector
// of nst super-tiles (128 elements each) is nst * kStepImg (576) bytes: dig[b * 4 + t][32] int8
// holds digit t of block b (nst * 512 bytes), then one BlockTab per block: s_b 2^-14, s_b 2^-21
// and -8 sum_j x_j.
struct alignas(16) BlockTab {
    float s14, s21, nbias, pad;
};

struct InputStage {
    const float* x;
    const float* res;
    const float* w_a;
    float eps_a;
    float scale;
    const float* w_n;
    float eps_n;
    float* x_out;
    Q6View table;
    const uint32_t* ids;
    const uint32_t* state;
    float emb_scale;
    const int8_t* dig;      // IN_DIGITS: the input's digit image
};

enum OutputKind : int {
    OUT_PLAIN = 0,  // y[r] = row sum
    OUT_GELU = 1,   // rows come in (gate, up) pairs: y[p] = f32(gelu_tanh(gate)) * up
    OUT_ADD = 2,    // y[r] = row sum + add[r]
};

struct Q4Args {
    Q4View w;      // the matrix (the gate matrix for OUT_GELU)
    Q4View w2;     // the up matrix for OUT_GELU
    InputStage in;
    float* y;
    const float* add;
    const uint32_t* state;  // session state (null for standalone use): exit at once when stopped
    uint32_t slices;        // waves splitting the super-tiles of a row tile (1, 2, 4 or 8)
    int8_t* dig_out;        // OUT_GELU: digit image of the output for the next GEMV (may be null)
};

// Session state words (device): position to consume next, sticky non-finite flag,
// stop flag (set by the head when it selects a stop id or sees non-finite logits;
// every kernel of a decode step returns immediately while it is set), and the
// number of stop ids.
// Session state words on the device.  The host uploads the first ST_HOST_WORDS; ST_EPOCH counts
// the step kernel's launches (the last workgroup out advances it) and tags the vectors that
// the step kernel publishes without a grid barrier.
enum { ST_POS = 0, ST_BAD = 1, ST_STOP = 2, ST_NSTOP = 3, ST_EPOCH = 4, ST_HOST_WORDS = 4, ST_WORDS = 5 };
constexpr uint32_t kMaxStopIds = 256;

// Per-step record the head writes to mapped host memory: id, non-finite flag, stop flag.
struct StepRecord {
    uint32_t id;
    uint32_t bad;
    uint32_t stop;
    uint32_t done;
};

struct HeadArgs {
    Q6View w;
    InputStage in;
    float* logits;          // may be null
    uint4* partial;         // one (value bits, id, bad, 0) per block
    uint32_t* counter;      // blocks done (reset to 0 by the last block)
    uint32_t* result;       // [id, bad] for the standalone head
    uint32_t* state;        // step mode: state words
    uint32_t* ids;          // step mode: ids[pos + 1] = argmax
    const uint32_t* stop_ids;  // step mode: state[ST_NSTOP] ids
    StepRecord* records;    // step mode: records[pos + 1] (mapped host memory)
};

struct AttnArgs {
    const float* q_raw;
    const float* k_raw;
    const float* v_raw;
    const float* q_norm;
    const float* k_norm;
    float q_eps, k_eps, v_eps;
    int v_norm;
    const double* inv_freq;  // head_width / 2
    uint16_t* kcache;        // fp16 [kv_heads][ring][head_width]
    uint16_t* vcache;
    uint32_t ring;
    uint32_t window;         // 0: global
    float scale;
    const uint32_t* state;   // non-null: position = state[ST_POS]
    uint32_t position;
    float* out;              // [q_heads][head_width]
    float* part;             // [tokens][kv_heads * group / G][cmax][G][attn_part_row(head_width)] (G: attention_block_heads)
    uint32_t* counters;      // [tokens][kv_heads * group / G], zero between launches
    int8_t* dig_out;         // digit image of `out` for the output projection (may be null)
    uint32_t cmax;
    uint32_t min_chunk;
    uint32_t kv_heads;
    uint32_t group;          // query heads per KV head
    int mode;                // AttnMode
    size_t in_stride;        // batch: floats between the tokens' q / k / v rows
    size_t out_stride;       // batch: floats between the tokens' outputs
    float* q_out;            // ATT_APPEND: the normalised, rotated queries [tokens][q_heads][head_width]
    // raw_parts > 0: the q / k / v rows are the split-K partials a batched GEMM left (its reduce
    // deferred): element i of token z's rows (i counted from q_raw; k_raw and v_raw point into the
    // same rows) is the sum, in split order, of raw_part[(k raw_tp + z) raw_prow + i], k < raw_parts
    const float* raw_part;
    uint32_t raw_parts, raw_prow, raw_tp;
    uint32_t tokens;         // set by launch_attention
    // the blocks of a slot share an XCD's L2 (workgroups b and b + 8 of a launch run on one XCD,
    // checked on this device by a probe launch): partials and tickets stay in that L2
    uint32_t xcd_local;
};

enum AttnMode : int {
    ATT_DECODE = 0,  // append the new K/V, attend
    ATT_APPEND = 1,  // append only
    ATT_ATTEND = 2,  // attend, every position's K/V already appended
};

// The C ABI's thread-local error message (af_last_error), set by every entry point that fails;
// returns code.
int set_error(int code, std::string msg);

// ---- batched prefill (batch.hip) ---------------------------------------------------------------
//
// Input image of T vectors of nb 32-element blocks for the batched GEMM, with the tokens padded to
// Tp = 16 ceil(T / 16) (padding tokens all zero): block b of vector t scaled by 2^(14 - e) (e =
// ilogb of the block's max |x|) as two fp16 halves, hi = f16(u) and lo = f16(u - hi):
//   hi  fp16 [nb][Tp][32], then lo fp16 [nb][Tp][32], then the scales 2^(e - 14) as float [nb][Tp]
constexpr uint32_t kBatchMax = 32;   // tokens per batch (crates/cuda-backend/src/batch.rs:10 MAX_BATCH)
constexpr uint32_t kVerifyMax = 16;  // tokens per speculative verification pass (batch.rs:13 MAX_VERIFY)

enum BatchInputKind : int { BI_PLAIN = 0, BI_RESID = 1, BI_EMBED = 2 };

struct BatchIn {
    int mode;               // BatchInputKind
    uint32_t T, K;          // vectors, elements (a multiple of 32)
    size_t stride;          // floats between the vectors of x, res and x_out
    const float* x;
    const float* res;
    const float* w_a;
    float eps_a;
    float scale;
    const float* w_n;       // null: no RMSNorm of the input
    float eps_n;
    float* x_out;
    float* snap;            // optional copy of x_out (layer outputs for tracing)
    size_t snap_stride;
    Q6View table;
    const uint32_t* ids;
    uint32_t pos0;          // BI_EMBED: vector t is row ids[pos0 + t]
    float emb_scale;
    // parts > 0: x comes from the split-K partial planes part[(k Tp + t) part_row + i] that
    // batch_gemm_kernel left (its reduce deferred), summed in split order: BI_RESID, planes
    // k < parts; BI_PLAIN without w_n, a gate/up pair: x = gelu(sum of gate planes 2 k) * (sum of up
    // planes 2 k + 1)
    const float* part;
    uint32_t parts;
    size_t part_row;
    int8_t* img;
};

struct BatchGemm {
    Q4View w, w2;           // w2: the up matrix of a gate/up pair
    const int8_t* img;      // input image of T vectors of w.blocks blocks (fp16 halves and scales)
    uint32_t T;
    float* y;               // y[t * y_stride + r], r < w.rows (gate/up: f32(gelu(gate)) * up)
    size_t y_stride;
    const float* add;       // optional residual added to y (same layout)
    float* part;            // split-K partials (batch_gemm_part_bytes)
    bool defer;             // no add: with a split-K plan of at most kDeferParts (a single matrix)
                            // or kDeferPairParts (a gate/up pair) splits, leave the partials for
                            // the input kernel of the next GEMM (no y)
};
constexpr uint32_t kDeferParts = 16, kDeferPairParts = 4;

// Attention of a batch over the KV cache after the append pass (batch_attention_kernel): the
// tokens' queries q[t][q_heads][D], token t at position pos0 + t seeing keys [max(0, pos0 + t + 1 -
// window), pos0 + t] (window 0: from 0).  Keys [klo, pos0 + T) go in nchunks chunks of span keys
// (a multiple of the kernel's sub-chunk); chunk partials (sum p v, max, sum p) per (token, head).
struct BatchAttn {
    const float* q;
    const uint16_t* kcache;
    const uint16_t* vcache;
    uint32_t ring, window, T, pos0, kv_heads, group;
    float scale;
    uint32_t klo, span, nchunks;
    float* part;             // [T q_heads][nchunks][D + 2]
    float* out;              // [T][out_stride]: head qh at qh D
    size_t out_stride;
};
constexpr uint32_t kBatchAttnChunks = 32;  // chunk partials per (token, head) at most

size_t batch_image_bytes(uint32_t blocks, uint32_t tokens);
hipError_t launch_batch_attention(BatchAttn a, uint32_t head_width, hipStream_t s);
size_t batch_gemm_part_bytes(uint32_t rows, uint32_t blocks, uint32_t tokens, bool gelu_pair);
hipError_t launch_batch_input(const BatchIn& in, hipStream_t s);
// Returns through parts the splits whose partials were left in a.part (0: y written).
hipError_t launch_batch_gemm(const BatchGemm& a, bool gelu_pair, hipStream_t s, uint32_t* parts = nullptr);

// ---- launchers (kernels.hip) -----------------------------------------------------------------
hipError_t launch_q4_gemv(const Q4Args& a, int in_kind, int out_kind, uint32_t out_rows, hipStream_t s);
hipError_t launch_head(const HeadArgs& a, int in_kind, uint32_t grid, hipStream_t s);
// The head (IN_RESID) over nv <= kHeadBatchMax hidden states at once, vector v's x and res at
// v vstride floats from a.in's; vector v's (id, bad) into a.result[2 v, 2 v + 1]; a.partial holds nv
// entries per workgroup.
constexpr uint32_t kHeadBatchMax = 4;
hipError_t launch_head_batch(const HeadArgs& a, uint32_t nv, uint32_t vstride, uint32_t grid, hipStream_t s);
hipError_t launch_attention(const AttnArgs& a, uint32_t group, uint32_t head_width, hipStream_t s,
                            uint32_t tokens = 1);
uint32_t attention_block_heads(uint32_t group, uint32_t head_width);
hipError_t launch_rmsnorm(const float* x, const float* w, float* y, uint32_t width, uint32_t vectors, float eps,
                          hipStream_t s);
hipError_t launch_resid(const InputStage& in, uint32_t width, float* y, hipStream_t s);
hipError_t launch_advance(uint32_t* state, hipStream_t s);
hipError_t launch_softcap(const float* x, float* y, size_t n, float cap, hipStream_t s);
hipError_t launch_zero_words(uint32_t* p, uint32_t n, hipStream_t s);
uint32_t head_grid(uint32_t rows);

constexpr uint32_t kAttnMinChunk = 32;
constexpr uint32_t kAttnShortChunks = 16;  // attention_kernel's short form: at most 16 chunks of 32
// A query head's chunk partial in attention_kernel's split-K scratch: D sums, the chunk's max and
// sum, padded so that every row starts on a 16-byte boundary.
__host__ __device__ constexpr uint32_t attn_part_row(uint32_t D) { return D + 4; }
constexpr uint32_t kAttnMaxChunkLen = 2048;
constexpr uint32_t kAttnMaxChunks = 64;  // cmax bound: capacity <= 64 * kAttnMaxChunkLen
constexpr uint32_t kHeadRows = 4;  // rows per wave iteration in the head kernel

// ---- persistent decode step (step.hip) ----------------------------------------------------------

// One layer as the step kernel reads it (device memory, one entry per layer).
struct StepLayer {
    Q4View qkv, o, gate, up, down;  // q, k (, v) rows stacked in qkv
    const float *input_norm, *q_norm, *k_norm, *post_attn, *ffn_norm, *post_ffn;
    const double* inv_freq;  // RoPE inverse frequencies (width / 2)
    uint16_t *kcache, *vcache;  // fp16 [kv_heads][ring][256]
    float input_eps, q_eps, k_eps, v_eps, post_attn_eps, ffn_eps, post_ffn_eps, layer_scale, scale;
    uint32_t q_heads, kv_heads, qn, kn, v_off, ring, window, v_norm;
    uint32_t chunks_max;  // attention chunks per KV head at most (StepArgs::cmax, or kStepWindowChunks)
};

// A windowed layer whose window fits this many staged chunks (StepArgs::stage_clen tokens each)
// splits its visible range into at most this many: past a few hundred positions half the grid
// then has no attention item and prefetches the gate/up records meanwhile.
constexpr uint32_t kStepWindowChunks = 16;

struct StepArgs {
    const StepLayer* layers;
    uint32_t n_layers, hidden, inter;
    Q6View table;  // tied embedding (layer 0 input)
    float emb_scale;
    const uint32_t* ids;
    uint32_t* state;
    float *X, *H, *QKV, *PROJ, *D;  // activations exchanged inside the launch
    uint32_t *QKVT, *PROJT, *DT;    // qkv, o-proj and down outputs as (value, tag) word pairs
    int8_t *att_img, *act_img;      // digit images of the o-proj (as tagged pieces) and down inputs
    float* part;                    // attention chunk partials
    uint32_t* counters;             // attention merge tickets, one per KV head
    uint32_t* bar;                  // grid barrier words (kStepBarBytes, zero between launches)
    const uint8_t* stream;          // every GEMV weight record of a step, one run per streaming wave
    const uint64_t* stream_off;     // [grid * kStepStreamWaves][2]: the byte range [start, end) of each
                                    // streaming wave's records of this launch's layers
    uint32_t cmax;                  // attention chunks per KV head (at most grid / kv_heads, and
                                    // what the merge can hold in LDS: step_merge_chunks)
    uint32_t advance;               // 1: move ST_POS on at the end (a step without the head)
    uint32_t xs_off;                // LDS byte offset of the residual prologue's staging (step_xs_offset)
    // LDS of an attention item (step_attn_layout): its "pre" part (RoPE frequencies, q/k norm
    // weights and the chunk's cached K/V rows, copied while the qkv phase runs) at attn_pre_off, clear
    // of the qkv phase's LDS; chunks of at most stage_clen tokens are staged there.
    uint32_t attn_pre_off, stage_clen;
    float* snap;                    // optional: layer outputs [n_layers][hidden] (the last by the head)
    uint64_t* clock;                // optional: [phases][kStepMarks][grid] timestamps (100 MHz), one
                                    // phase per barrier interval (see StepMark)
    uint32_t fail_phase;            // a phase whose opening grid barrier waits for one arrival too
                                    // many, so that it ends in the barrier's own time-out (a host-set
                                    // test of the fall-back path); ~0u: none
    uint32_t xcd_local;             // 1: head group h's qkv rows, attention items and chunk partials all
                                    // live on one XCD (workgroups b with b % 8 == h) and are exchanged
                                    // through that XCD's L2 (step_qkv_tile, step_attn_chunk)
    // Values handed over by launch layer l carry the tag epoch * tag_stride + 1 + tag_base + l (epoch:
    // state word ST_EPOCH, one more per launch; tag_base + n_layers <= tag_stride), so that no tag
    // repeats across the launches of a session.
    uint32_t tag_stride, tag_base;
    // Non-null: the launch's layer 0 follows a layer run by the per-operation kernels and takes its
    // input from D and H as plain floats, with that layer's post-FFN norm and scale.
    const float* prev_post_ffn;
    float prev_post_ffn_eps, prev_scale;
};

// XCD-local layout (StepArgs::xcd_local): eight KV heads of two query heads each, a 256-workgroup
// grid whose workgroups b and b + 8 share an XCD (workgroup b on XCD (x0 + b) % 8, x0 varying from
// launch to launch; verified at session open by step_xcd_map).  Head group
// h = b % 8 owns 64 qkv tiles (its two query heads' 32, its K head's 16, its V head's 16), two per
// workgroup of rank r = b / 8; its attention chunk c runs on workgroup 8 (31 - c) + h.
constexpr uint32_t kXcds = 8;

// Row tile of qkv unit k (0 or 1) of workgroup b: b + k grid, or in the XCD-local layout the head
// group's tile 2 r + k (qn_tiles = query rows / 16, kn_tiles = key rows / 16).
__host__ __device__ inline uint32_t step_qkv_tile(uint32_t b, uint32_t k, uint32_t grid, uint32_t xl, uint32_t qn_tiles,
                                                  uint32_t kn_tiles) {
    if (!xl) return b + k * grid;
    const uint32_t h = b % kXcds, j = 2 * (b / kXcds) + k;
    const uint32_t gq = qn_tiles / kXcds, gk = kn_tiles / kXcds;  // tiles per head group
    if (j < gq) return h * gq + j;
    if (j < gq + gk) return qn_tiles + h * gk + (j - gq);
    return qn_tiles + kn_tiles + h * gk + (j - gq - gk);
}

// Timeline marks of a phase (workgroup's thread 0): start (barrier departure or kernel start),
// inputs staged, digit image built, weights streamed, outputs stored, arrival at the closing
// barrier (or kernel end), the pre-barrier work of the next phase done, and (wave 1) its weight
// records consumed.  An attention phase marks: q/k/v staged, chunk partial computed, partial
// published (ticket taken), merge done.
enum StepMark { M_START = 0, M_STAGED, M_DIGITS, M_STREAMED, M_STORED, M_ARRIVE, M_PRE, M_CONSUMED, kStepMarks = 8 };

constexpr uint32_t kStepMaxClen = 2048;   // tokens per attention chunk
constexpr uint32_t kStepMaxChunks = 256;  // chunks per KV head
constexpr uint32_t kStepMaxUnits = 2;     // GEMV row units per workgroup (16 rows, 32 for gate/up)
constexpr size_t kStepBarBytes = 32 * 10 * 4;

// Weight stream of the step kernel.  A GEMV phase's rows are grouped in units (one 16-row tile;
// for gate/up, tiles 2u, 2u + 1 of gate then of up: T = 4 tile streams per unit); workgroup b
// takes units b, b + grid, ... (at most kStepMaxUnits), and its super-tiles, flattened as
// f = (unit, tile stream, super-tile), go to streaming wave w = 1..7 for f = w - 1, w + 6, ...
// Each (workgroup, wave) reads one contiguous run of records, every phase of every layer in
// consume order; a record is one super-tile of one row tile: the 1024 code bytes of the tiled
// Q4View layout followed by its 128 scale bytes.
constexpr uint32_t kStepStreamWaves = 7;
constexpr uint32_t kStepRecord = 1152;
constexpr uint32_t kStepImg = 576;  // digit image bytes per super-tile: 512 digits + 4 BlockTab entries
constexpr uint32_t kStepStreamPad = 64 * kStepRecord;  // readable bytes after the last run (ring over-read)

__host__ __device__ inline uint32_t step_units(uint32_t units, uint32_t b, uint32_t grid) {
    if (units <= b) return 0u;
    const uint32_t n = (units - b + grid - 1) / grid;
    return n < kStepMaxUnits ? n : kStepMaxUnits;
}
// Records of wave w (1..7) of workgroup b in a phase of `units` units, T tile streams, nst super-tiles.
__host__ __device__ inline uint32_t step_wave_records(uint32_t units, uint32_t T, uint32_t nst, uint32_t b,
                                                      uint32_t grid, uint32_t w) {
    const uint32_t fe = step_units(units, b, grid) * T * nst;
    return fe > w - 1 ? (fe - (w - 1) + kStepStreamWaves - 1) / kStepStreamWaves : 0u;
}

// Floats per attention chunk partial of the step kernel: GQ query heads of 256 unnormalised
// outputs plus their softmax max and sum, padded to a multiple of 4 so that every chunk starts
// on a 16-byte boundary and is stored and copied in whole 16-byte pieces (GQ * 258 alone is not a
// multiple of 4 for odd GQ).
__host__ __device__ constexpr uint32_t step_part_stride(uint32_t group) { return (group * (256u + 2u) + 3u) & ~3u; }

size_t step_lds_bytes(uint32_t hidden, uint32_t inter, uint32_t q_dim, uint32_t group);
// Where an attention item's "pre" LDS part goes and how many tokens a chunk stages there.
void step_attn_layout(uint32_t hidden, uint32_t inter, uint32_t q_dim, uint32_t group, uint32_t* pre_off,
                      uint32_t* stage_clen);
uint32_t step_xs_offset(uint32_t hidden, uint32_t inter, uint32_t q_dim);
uint32_t step_merge_chunks(uint32_t group, size_t lds);  // chunk partials one merge holds in LDS
hipError_t step_max_grid(uint32_t group, size_t lds, uint32_t* grid);
hipError_t launch_step(const StepArgs& a, uint32_t group, uint32_t grid, size_t lds, hipStream_t s);
// Fills the weight stream (StepArgs::stream at stream_off) from the layers' tiled Q4View matrices.
hipError_t launch_stream_repack(const StepLayer* layers, uint32_t n_layers, uint32_t grid, uint32_t xcd_local,
                                uint8_t* stream, const uint64_t* stream_off, hipStream_t s);
// The XCD each workgroup of a `grid`-workgroup launch runs on (hardware register XCC_ID), one word
// per workgroup into xcc (device memory).
hipError_t step_xcd_map(uint32_t grid, uint32_t* xcc, hipStream_t s);

}  // namespace af
