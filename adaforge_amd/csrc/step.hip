// Persistent decode step for gfx950 (MI355X): all layers of one decode step in one launch of one
// 512-thread workgroup per CU.  Per layer it runs five phases: qkv GEMV (residual + RMSNorm
// prologue), GQA attention over the fp16 KV cache (split-K, merged by the last chunk of each KV
// head), o-proj GEMV, fused gate/up GEMV with tanh-GELU, down GEMV.  Down opens with a grid
// barrier; the other phases poll their inputs, which their producers store with tags.
//
// Why one launch: a layer's five dependent kernels each pay a dispatch, a ramp and a drain,
// and their weight streams cannot start before the previous kernel ends.  Here the weights of
// the next phase, which do not depend on any activation, are requested before each phase
// boundary, so HBM keeps streaming while the boundary and the next phase's input prologue
// resolve.
//
// Wave roles: wave 0 of every workgroup never streams weights: it runs the grid barrier, the
// next phase's early copies and the output stores, while waves 1-7 stream the weights, each
// from its own contiguous run of weight records.  At a phase start all eight waves poll or copy
// the phase's input into LDS (a streaming wave's weight loads still in flight were issued
// before), and the input prologue (norms, int8 digit planes) runs on all 512 threads
// from LDS.
//
// Coherence: the eight XCDs have private L2 caches.  Activations exchanged between workgroups
// inside the launch are written and read with agent-scope coherent accesses (sc1), the grid
// barrier uses agent-scope atomics, and a store is waited for (s_waitcnt vmcnt(0)) before the
// barrier arrival that publishes it; a tagged value carries its tag in the same store.
// Weights, norm vectors and the KV cache rows read here were written before the launch began.
#include "device.h"

namespace af {

namespace {

constexpr uint32_t kThreads = 512;
constexpr uint32_t kStreamWaves = kStepStreamWaves;  // waves 1..7 stream weights
constexpr int kRing = 8;              // weight records in flight per streaming wave
constexpr int kSC1 = 16;              // cache policy: agent-scope coherent access (through to the
                                      // memory side, where every XCD's accesses meet)
constexpr int kSC0 = 1;               // cache policy (stores): workgroup scope, into the XCD's L2;
                                      // other workgroups of the XCD read it with kNT loads, which
                                      // miss their CU's L1 and hit that L2 (measured round trip
                                      // between two workgroups of one XCD: 0.42 us, against 1.04 us
                                      // through the memory side with kSC1)
constexpr int kNT = 2;                // cache policy: non-temporal (weights are read once per step; a
                                      // non-temporal load also misses the CU's L1)
constexpr int kVmWait = 0x0F70;       // s_waitcnt vmcnt(0) with expcnt / lgkmcnt unconstrained
constexpr uint32_t kSpinLimit = 1u << 21;
constexpr uint32_t kMaxUnits = kStepMaxUnits;
constexpr uint32_t kMaxT = 4;         // tile streams per unit (gate/up: 2 tiles of 2 matrices)

// Barrier words, 128 bytes apart: [0] groups done, [32 (g + 1)] arrivals of group g (g < 8,
// workgroups b with b % 8 == g, which share an XCD), [32 * 9] exits.
constexpr uint32_t kBarAll = 0, kBarExit = 32 * 9;

typedef __attribute__((address_space(3))) void* lds_ptr;

// The layer table is read through the constant address space: uniform scalar loads.  Through a
// generic pointer the compiler would use vector loads (it cannot rule out that the kernel's
// stores alias the table) and wait for every load in flight, weight prefetch included.
typedef const __attribute__((address_space(4))) StepLayer CLayer;
typedef const __attribute__((address_space(4))) Q4View CQ4View;
__device__ __forceinline__ CLayer& layer_at(const StepArgs& a, uint32_t l) {
    return ((CLayer*)(a.layers))[l];
}

__device__ __forceinline__ __amdgpu_buffer_rsrc_t rsrc(const void* p) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(p), 0, 0x7FFFFFFF, 0x00020000);
}
__device__ __forceinline__ void stc(void* base, uint32_t off, uint32_t v) {
    __builtin_amdgcn_raw_buffer_store_b32(v, rsrc(base), off, 0, kSC1);
}
__device__ __forceinline__ void stc8(void* base, uint32_t off, v2u v) {
    __builtin_amdgcn_raw_buffer_store_b64(v, rsrc(base), off, 0, kSC1);
}
__device__ __forceinline__ void stc16(void* base, uint32_t off, v4u v) {
    __builtin_amdgcn_raw_buffer_store_b128(v, rsrc(base), off, 0, kSC1);
}
template <int Pol>
__device__ __forceinline__ void st8p(void* base, uint32_t off, v2u v) {
    __builtin_amdgcn_raw_buffer_store_b64(v, rsrc(base), off, 0, Pol);
}
template <int Pol>
__device__ __forceinline__ void st16p(void* base, uint32_t off, v4u v) {
    __builtin_amdgcn_raw_buffer_store_b128(v, rsrc(base), off, 0, Pol);
}
__device__ __forceinline__ void wait_vm() { __builtin_amdgcn_s_waitcnt(kVmWait); }

// threadIdx.x through an empty asm, read once per phase: the per-lane values derived from it are
// then computed inside the phase that uses them.  Hoisted out of the phase loop (the thread index
// is loop-invariant) they would hold registers through every phase, the weight ring's included.
__device__ __forceinline__ uint32_t tix() {
    uint32_t t = threadIdx.x;
    asm volatile("" : "+v"(t));
    return t;
}

// Wave-level global -> LDS copy of `bytes` (a multiple of 16) with coherent loads; the caller
// waits with wait_vm().
__device__ __forceinline__ void dma(const void* src, uint32_t bytes, uint8_t* lds, uint32_t lane) {
    for (uint32_t off = 0; off < bytes; off += 1024) {
        if (off + lane * 16 < bytes)
            __builtin_amdgcn_global_load_lds(static_cast<const uint8_t*>(src) + off + lane * 16,
                                             (lds_ptr)(lds + off), 16, 0, kSC1);
    }
}

// The same copy split over the workgroup's 8 waves (wave w takes every 8th KB), so that one
// wave's issue rate does not bound it; each wave waits for its own part.  Pol: the loads' cache
// policy (kSC1, or kSC0 for data another workgroup of this XCD wrote).
template <int Pol = kSC1>
__device__ __forceinline__ void dma_all(const void* src, uint32_t bytes, uint8_t* lds, uint32_t wave, uint32_t lane) {
    for (uint32_t off = wave * 1024; off < bytes; off += 8 * 1024) {
        if (off + lane * 16 < bytes)
            __builtin_amdgcn_global_load_lds(static_cast<const uint8_t*>(src) + off + lane * 16,
                                             (lds_ptr)(lds + off), 16, 0, Pol);
    }
}

// The same copy split into 1 KB stripes over n waves (this one is number i < n).
__device__ __forceinline__ void dma_part(const void* src, uint32_t bytes, uint8_t* lds, uint32_t i, uint32_t n,
                                         uint32_t lane) {
    for (uint32_t off = i * 1024; off < bytes; off += n * 1024) {
        if (off + lane * 16 < bytes)
            __builtin_amdgcn_global_load_lds(static_cast<const uint8_t*>(src) + off + lane * 16,
                                             (lds_ptr)(lds + off), 16, 0, kSC1);
    }
}

// ---- grid barrier -------------------------------------------------------------------------------

struct Grid {
    uint32_t* bar;
    uint32_t k;       // barriers passed in this launch
    uint32_t p;       // phase (of the timeline) the workgroup is in
    int* ok;          // LDS flag
    uint64_t* clock;  // optional timeline (StepArgs::clock)
};

// Thread 0 only.
__device__ __forceinline__ void stamp_at(const Grid& g, uint32_t phase, uint32_t mark) {
    if (g.clock) g.clock[((size_t)phase * kStepMarks + mark) * gridDim.x + blockIdx.x] = wall_clock64();
}
// Wave 0 stores (every lane the same value to the same word): a branch on the wave index is
// uniform, where one on the thread index would make the phase loop's control flow divergent.
__device__ __forceinline__ void stamp(const Grid& g, uint32_t mark) {
    if (wave_id() == 0) stamp_at(g, g.p, mark);
}

// All threads call it.  Returns false (in every thread) if the barrier did not complete within
// the spin limit, which only a launch without co-resident workgroups could cause.  With `lead`
// the workgroup first waits for all its waves (their stores are waited for before they arrive);
// without it, wave 0 alone has published the phase's outputs and arrives for the workgroup.
// `extra` (0 or 1) raises the count waited for beyond what the grid can reach: the host's test of
// the time-out (StepArgs::fail_phase).
__device__ __forceinline__ bool grid_sync(Grid& g, bool lead, uint32_t extra) {
    if (lead) __syncthreads();
    if (threadIdx.x == 0) {
        stamp_at(g, g.p, M_ARRIVE);
        const uint32_t per = gridDim.x / 8, grp = blockIdx.x & 7, k = g.k + 1;
        const uint32_t old =
            __hip_atomic_fetch_add(g.bar + 32 * (1 + grp), 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        if (old + 1 == k * per) __hip_atomic_fetch_add(g.bar + kBarAll, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        uint32_t spins = 0;
        int ok = 1;
        while (__hip_atomic_load(g.bar + kBarAll, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) < 8 * k + extra) {
            __builtin_amdgcn_s_sleep(1);
            if (++spins > kSpinLimit) {
                ok = 0;
                break;
            }
        }
        *g.ok = ok;
        stamp_at(g, g.p + 1, M_START);
    }
    __syncthreads();
    ++g.k;
    ++g.p;
    return __builtin_amdgcn_readfirstlane(*g.ok) != 0;  // uniform: keeps the phase loop scalar
}

// A phase boundary without a grid barrier: the next phase's input carries its own tags
// (poll_tagged).  Only the timeline moves on.
__device__ __forceinline__ void tagged_boundary(Grid& g) {
    if (wave_id() == 0) {
        stamp_at(g, g.p, M_ARRIVE);
        stamp_at(g, g.p + 1, M_START);
    }
    ++g.p;
}

// Last workgroup out resets the barrier words for the next launch; with `advance` it also moves
// the session position (a step without the head), unless a workgroup failed: then the position
// stays at the failed step, which the host runs again on the per-operation kernels.  A failing
// workgroup's state stores (agent scope: through to the memory side) complete before its exit
// arrival, and the last arrival reads them with an agent-scope load after its own arrival, so no
// L2 write-back or invalidation (an acquire-release at device scope) is needed.
__device__ __forceinline__ void grid_exit(Grid& g, uint32_t* state, bool advance, bool failed) {
    __syncthreads();
    if (threadIdx.x == 0) {
        stamp_at(g, g.p, M_ARRIVE);
        if (failed) {
            __hip_atomic_store(state + ST_BAD, 2u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            __hip_atomic_store(state + ST_STOP, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
        wait_vm();
        const uint32_t old = __hip_atomic_fetch_add(g.bar + kBarExit, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        if (old == gridDim.x - 1) {
            for (uint32_t i = 0; i < 10; ++i)
                __hip_atomic_store(g.bar + 32 * i, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            const bool any_failed =
                __hip_atomic_load(state + ST_BAD, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == 2u;
            if (advance && !any_failed) state[ST_POS] += 1u;
            state[ST_EPOCH] += 1u;  // read by the next launch, which the end of this one orders
        }
    }
}

// ---- GEMV phases --------------------------------------------------------------------------------

// Shape of a GEMV phase: units of T tile streams of nst super-tiles (StepArgs::stream).
struct Shape {
    uint32_t nst, T, units;
};

// Row partials of a GEMV phase in LDS: part[(k kMaxT + ts) 8 + wave][16 rows], a wave's sums over
// its super-tiles of tile stream ts of unit k.
constexpr uint32_t kPart = kMaxUnits * kMaxT * 8 * 16;

__device__ __forceinline__ void zero_part_lds(float* part, uint32_t tid) {
    for (uint32_t i = tid; i < kPart; i += kThreads) part[i] = 0.0f;
}

__device__ __forceinline__ float part_sum(const float* part, uint32_t k, uint32_t ts, uint32_t r) {
    const float* p = part + (k * kMaxT + ts) * 8 * 16 + r;
    float v = p[16];  // wave 0 never streams
#pragma unroll
    for (int w = 2; w < 8; ++w) v += p[16 * w];
    return v;
}




// A streaming wave's weight records: a ring of kRing in registers, refilled from the wave's run
// as each is consumed, across phase (and layer) boundaries: the next phase's first records are
// in flight while this one finishes and during the boundary and prologue in between.  Slot
// `slot` holds the next record to consume.
static_assert(kRing * kStepRecord <= kStepStreamPad, "stream padding below the ring's over-read");

struct Ring {
    v4u code[kRing];
    uint32_t scale[kRing];
    uint32_t base_lo, base_hi, len;  // the wave's run (wave-uniform)
    uint32_t soff;                   // byte offset of the next record to request
    uint32_t slot;
};

// Buffer view of the wave's run.  Built from readfirstlane values so that the descriptor is known
// to be wave-uniform (scalar registers); readfirstlane returns int, so each half is taken as
// unsigned before the halves are joined.  The record offset goes in soffset, which the range
// check does not cover: the ring's last refills read up to kRing records past the run, which the
// allocation's padding (kStepStreamPad) keeps inside it.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t ring_rsrc(const Ring& r) {
    const uint64_t p = ((uint64_t)(uint32_t)__builtin_amdgcn_readfirstlane(r.base_hi) << 32) |
                       (uint64_t)(uint32_t)__builtin_amdgcn_readfirstlane(r.base_lo);
    return __builtin_amdgcn_make_buffer_rsrc(reinterpret_cast<void*>(p), 0, (int)__builtin_amdgcn_readfirstlane(r.len),
                                             0x00020000);
}

// Records a streaming wave of a workgroup without an attention item pulls through the caches during
// the attention phase: those after its ring, i.e. the rest of o-proj, gate/up and the first of down.
// One 4-byte DMA per 128-byte line into a dword of an LDS slot that nothing reads (a DMA needs an
// LDS destination and no registers): the miss fetches the whole line into L2 and the Infinity
// Cache, so the wave's own ring loads of it later return at cache latency, while HBM would
// otherwise idle; moving every byte to the CU instead (1 KB per instruction) cost 32 times the
// cache-to-CU traffic and 8 times the instructions for the same gain.
constexpr uint32_t kPrefetchRecords = 30;
constexpr uint32_t kPrefetchLine = 128;
static_assert((kRing + kPrefetchRecords) * kStepRecord <= kStepStreamPad, "stream padding below the prefetch");

__device__ __forceinline__ void prefetch_records(const Ring& r, uint8_t* sink, uint32_t lane) {
    const uint64_t base = ((uint64_t)r.base_hi << 32) | r.base_lo;
    const uint8_t* src = reinterpret_cast<const uint8_t*>(base) + r.soff;
    constexpr uint32_t kBytes = kPrefetchRecords * kStepRecord;
    for (uint32_t i = 0; i < kBytes; i += 64 * kPrefetchLine)
        if (i + lane * kPrefetchLine < kBytes)  // inside the window the padding covers
            __builtin_amdgcn_global_load_lds(src + i + lane * kPrefetchLine, (lds_ptr)sink, 4, 0, 0);
}

__device__ __forceinline__ void ring_fill(Ring& r, const __amdgpu_buffer_rsrc_t& rs, int u, uint32_t lane) {
    r.code[u] = __builtin_amdgcn_raw_buffer_load_b128(rs, lane * 16, r.soff, kNT);
    r.scale[u] = __builtin_amdgcn_raw_buffer_load_b16(rs, 1024 + lane * 2, r.soff, kNT);
    r.soff += kStepRecord;
}

// Rotates the ring so that the next record to consume is in slot 0 (register moves only; the
// caller has waited for every load in flight).
template <int S>
__device__ __forceinline__ void ring_rotate_by(Ring& r) {
    v4u c[kRing];
    uint32_t q[kRing];
#pragma unroll
    for (int i = 0; i < kRing; ++i) {
        c[i] = r.code[(i + S) % kRing];
        q[i] = r.scale[(i + S) % kRing];
    }
#pragma unroll
    for (int i = 0; i < kRing; ++i) {
        r.code[i] = c[i];
        r.scale[i] = q[i];
    }
}
template <int S = 1>
__device__ __forceinline__ void ring_rotate(Ring& r) {
    if constexpr (S < kRing) {
        if (r.slot == S) ring_rotate_by<S>(r);
        else ring_rotate<S + 1>(r);
    }
}

// Per-lane constants of the matrix-core step.  The MFMA computes D = A B with A = the input's
// digit planes (row m = 4 g + t: digit t of block g of the super-tile; k-group g of lane
// (m, g) holds the block's 16 digits when g == m / 4, zeros otherwise) and B = the 16 code
// bytes of (block g, row r) at lane 16 g + r (low nibbles in one MFMA against elements 0..15,
// high nibbles in a second against 16..31).  Lane l then holds D[4 q + i][r] for digit i of
// block q = l / 16 and row r = l % 16, which it folds with its one block scale d(r, q).
struct LaneK {
    uint32_t aoff;  // active A lanes: byte offset of their digit plane within a super-tile image
    uint32_t q16;   // block entry of the lane's output block within a super-tile
    bool aon;
};

__device__ __forceinline__ LaneK lane_k(uint32_t lane) {
    LaneK k;
    k.aon = ((lane & 15) >> 2) == (lane >> 4);
    k.aoff = (lane & 15) * 32;
    k.q16 = (lane >> 4) * 16;
    return k;
}

// LDS byte addresses of a phase's record operands for this lane: the digit planes of super-tile st
// at a0 + st * am (am = 0 and a0 = the zero block for inactive A lanes) and the lane's BlockTab
// entry at t0 + 64 st.
struct LaneAddr {
    uint32_t a0, am, t0;
};

__device__ __forceinline__ LaneAddr lane_addr(const uint8_t* img, const v4i* zero, uint32_t nst, const LaneK& lk) {
    LaneAddr a;
    a.a0 = lk.aon ? lds_addr(img) + lk.aoff : lds_addr(zero);
    a.am = lk.aon ? 512u : 0u;
    a.t0 = lds_addr(img) + nst * 512 + lk.q16;
    return a;
}

__device__ __forceinline__ void split_codes(const v4u c, v4i& bl, v4i& bh) {
    constexpr uint32_t M = 0x0F0F0F0Fu;
    bl = v4i{(int)(c.x & M), (int)(c.y & M), (int)(c.z & M), (int)(c.w & M)};
    bh = v4i{(int)((c.x >> 4) & M), (int)((c.y >> 4) & M), (int)((c.z >> 4) & M), (int)((c.w >> 4) & M)};
}

// Position of a wave's next record in a GEMV phase (wave-uniform).  The wave's super-tiles are f =
// wave - 1, wave + 6, ... (flattened over unit k, tile stream ts, super-tile st) below fe; a run is
// its super-tiles of one (k, ts).  A step of 7 super-tiles (7 = dseg nst + dst) advances st by dst
// and the run by dseg, or by dseg + 1 when st wraps; the run's row sums go to part[prow + r].
struct Cursor {
    uint32_t st, prow;      // super-tile, part offset of the run
    uint32_t nst, dst;
    uint32_t pstep0, pstep1;  // prow advance without / with a wrap
    bool end0;                // a step without a wrap leaves the run (nst < 7)
};

__device__ __forceinline__ Cursor cursor_start(uint32_t nst, uint32_t T, uint32_t wave) {
    Cursor c;
    const uint32_t f = wave - 1;
    // f < 7: with 8 or more super-tiles per run (every phase of the models here) no division
    const uint32_t seg = nst >= 8 ? 0u : f / nst, dseg = nst >= 8 ? 0u : 7 / nst;
    const uint32_t pstep = T == 1 ? kMaxT * 8 * 16 : 8 * 16;  // one (k, ts) further; T is 1 or 4
    c.nst = nst;
    c.dst = nst >= 8 ? 7u : 7 % nst;
    c.pstep0 = dseg * pstep;
    c.pstep1 = (dseg + 1) * pstep;
    c.end0 = dseg != 0;
    c.st = f - seg * nst;
    c.prow = seg * pstep + wave * 16;
    return c;
}

// One record of slot u: two int8 MFMAs against the digit image, the fold into the lane's partial,
// the refill of the slot (with Fill), and at the run's end its row sums into part (a uniform
// branch: every lane of a row writes the same value) and a fresh partial.
template <bool Fill = true>
__device__ __forceinline__ void consume_one(Ring& r, const __amdgpu_buffer_rsrc_t& rs, int u, Cursor& c, float& acc,
                                            const LaneAddr& la, float* part, uint32_t lane) {
    const uint32_t s1 = c.st + c.dst, s2 = s1 - c.nst;
    const bool wrap = s1 >= c.nst;
    const bool last = wrap || c.end0;  // the run's last record (the phase's last: see consume_phase)
    const uint32_t pa = la.a0 + __umul24(c.st, la.am);  // full-rate 24-bit multiply (st < 2^24, am <= 512)
    const v4i a0 = lds_at<v4i>(pa), a1 = lds_at<v4i>(pa + 16);
    const v4f tb = lds_at<v4f>(la.t0 + c.st * 64);  // BlockTab: s14, s21, nbias
    const v4i zero4 = {0, 0, 0, 0};
    v4i bl, bh;
    split_codes(r.code[u], bl, bh);
    v4i d = __builtin_amdgcn_mfma_i32_16x16x64_i8(a0, bl, zero4, 0, 0, 0);
    d = __builtin_amdgcn_mfma_i32_16x16x64_i8(a1, bh, d, 0, 0, 0);
    // 2^14 D0 + 2^7 D1 + D2 is exact in int32 (|D_t| <= 32 * 15 * 64)
    const int I = (d[0] << 14) + (d[1] << 7) + d[2];
    float in = fmaf((float)I, tb.x, tb.z);
    in = fmaf((float)d[3], tb.y, in);
    acc = fmaf(h2f((uint16_t)r.scale[u]), in, acc);
    if constexpr (Fill) ring_fill(r, rs, u, lane);  // after the last use of the slot's registers
    if (last) {
        part[c.prow + (lane & 15)] = row_total(acc);
        acc = 0.0f;
    }
    c.prow += wrap ? c.pstep1 : c.pstep0;
    c.st = wrap ? s2 : s1;
}

// The phase's last record ends its run whether or not the next step wraps: its row sums, unless
// that record already wrote them (acc was reset).  c has advanced past the record.
__device__ __forceinline__ void flush_last(float acc, const Cursor& c, float* part, uint32_t lane) {
    // the run of the last record: prow before the step (no wrap: pstep0 was added)
    if (c.st >= c.dst && !c.end0) part[c.prow + (lane & 15)] = row_total(acc);
}

// A streaming wave's partials are all in part: +64 on the workgroup's LDS counter (every lane adds
// one), ordered after the wave's LDS writes.
__device__ __forceinline__ void signal_done(uint32_t* done) {
    __hip_atomic_fetch_add(done, 1u, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_WORKGROUP);
}

// Consumes this wave's records of a GEMV phase (fe = the workgroup's flattened super-tiles), leaves
// its partials in part and signals `done`.  img: the phase's digit image in LDS.  The ring arrives
// with its next record in slot 0 (the caller rotated it at the end of the previous phase).
// * When the ring holds every record of the phase, they are consumed first and the slots are
//   refilled after the signal: a refill cannot issue while the memory system is saturated, and
//   that wait then delays neither the records nor the phase's epilogue.
// * Otherwise whole rounds of kRing records run without an exit test (exact waits: slot u's loads
//   are followed by those of the kRing - 1 slots after it), then a tail of fewer than kRing.
__device__ __forceinline__ void consume_phase(Ring& r, uint32_t nst, uint32_t T, uint32_t fe, const uint8_t* img,
                                              const v4i* zero, float* part, uint32_t wave, uint32_t lane,
                                              const LaneK& lk, uint32_t* done) {
    if (wave - 1 >= fe) return;
    wait_vm();  // every record in flight was requested before this phase began
    const __amdgpu_buffer_rsrc_t rs = ring_rsrc(r);
    r.soff = __builtin_amdgcn_readfirstlane(r.soff);
    const uint32_t total = (fe - (wave - 1) + 6) / 7;
    const LaneAddr la = lane_addr(img, zero, nst, lk);
    Cursor c = cursor_start(nst, T, wave);
    float acc = 0.0f;
    if (total <= kRing) {
#pragma unroll
        for (int u = 0; u < kRing; ++u)
            if ((uint32_t)u < total) consume_one<false>(r, rs, u, c, acc, la, part, lane);
        flush_last(acc, c, part, lane);
        signal_done(done);
#pragma unroll
        for (int u = 0; u < kRing; ++u)
            if ((uint32_t)u < total) ring_fill(r, rs, u, lane);
        r.slot = total % kRing;
        return;
    }
    for (uint32_t i = total / kRing; i; --i) {
#pragma unroll
        for (int u = 0; u < kRing; ++u) consume_one(r, rs, u, c, acc, la, part, lane);
    }
    const uint32_t rem = total % kRing;
#pragma unroll
    for (int u = 0; u < kRing - 1; ++u)
        if ((uint32_t)u < rem) consume_one(r, rs, u, c, acc, la, part, lane);
    r.slot = rem;
    flush_last(acc, c, part, lane);
    signal_done(done);
}

// Input prologue of a GEMV phase: LDS layout [digit image nst * kStepImg] ... and, at StepArgs::xs_off
// (above the largest image of any phase, so the next phase's norm weights can be copied in while
// this phase's image is in use), [x K][res K][w_a K][w_n K] (floats).  Every wave stages, every
// thread then builds the digit image.
enum StageKind { S_EMBED = 0, S_RESID = 1, S_DIGITS = 2, S_TDIGITS = 3 };  // S_TDIGITS: tagged (poll_image)

struct Stage {
    const float *res, *w_a, *w_n;
    const uint32_t* xt;   // S_RESID: the input as (value, tag) word pairs (poll_tagged); S_TDIGITS: the
                          // tagged digit image (poll_image)
    const float* xf;      // S_RESID instead of xt: the input as plain floats, written before the launch
    uint32_t tag;         // the tag of the input's current values
    float eps_a, eps_n, scale;
    const int8_t* dig;    // S_DIGITS
    float* x_out;         // S_EMBED / S_RESID: the residual, written by workgroup 0
    float* snap;          // optional copy of x_out
};

// A vector handed from one GEMV phase to the next without a grid barrier: element i is the word
// pair (value, tag) at 8 i, stored by its producer with one 8-byte store, and tag identifies the
// launch and layer that wrote it.  Every thread reads 16-byte pieces tid, tid + 512, .. (K <= 4096:
// at most 4) and re-reads the pieces whose tags are not yet `tag`; a current piece's two values
// go to xs.  A pair is never overwritten before every workgroup has read it: the grid barriers
// between its consumer phase and its producer's next turn order the two.  Returns false (in the
// whole wave) if the wave's pieces did not all become current within the spin limit.
constexpr uint32_t kPollLimit = 1u << 20;

__device__ __forceinline__ bool poll_tagged(const uint32_t* src, uint32_t K, uint32_t tag, float* xs, uint32_t tid) {
    const __amdgpu_buffer_rsrc_t rs = rsrc(src);
    const uint32_t n = K / 2;
    uint32_t need = 0;
#pragma unroll
    for (int i = 0; i < 4; ++i)
        if (tid + kThreads * i < n) need |= 1u << i;
    for (uint32_t spins = 0;; ++spins) {
        v4u v[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            v[i] = v4u{0u, 0u, 0u, 0u};
            if (need >> i & 1) v[i] = __builtin_amdgcn_raw_buffer_load_b128(rs, (tid + kThreads * i) * 16, 0, kSC1);
        }
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            if ((need >> i & 1) && v[i].y == tag && v[i].w == tag) {
                reinterpret_cast<v2u*>(xs)[tid + kThreads * i] = v2u{v[i].x, v[i].z};
                need &= ~(1u << i);
            }
        }
        if (__builtin_amdgcn_ballot_w64(need != 0) == 0) return true;
        if (spins >= kPollLimit) return false;
        __builtin_amdgcn_s_sleep(1);
    }
}

// A digit image handed over without a grid barrier: its 8-byte word i (bytes lo, hi) is the
// 16-byte piece (lo, tag, hi, tag) at 16 i of the tagged image.  Wave w polls the pieces of chunks
// j = w, w + 8, .. (64 pieces each, piece j 64 + lane in lane `lane`), re-reads the pieces whose
// tags are not yet current, and writes a current piece's word to the image in LDS.  Up to 6 chunks
// per wave the pieces are loaded into registers; a larger image goes through LDS staging
// stg + 1024 j (one DMA per chunk), which costs an LDS round trip per poll.  Returns false (in the
// whole wave) if its pieces did not become current within the spin limit.
__device__ __forceinline__ bool poll_image(const uint32_t* src, uint32_t bytes, uint32_t tag, uint8_t* img, uint8_t* stg,
                                           uint32_t wave, uint32_t lane) {
    const uint32_t n = bytes / 8, nj = (n + 63) / 64;
    uint32_t need = 0;
    for (uint32_t i = 0, j = wave; j < nj; ++i, j += 8)
        if (j * 64 + lane < n) need |= 1u << i;
    if (nj <= 8 * 6) {
        const __amdgpu_buffer_rsrc_t rs = rsrc(src);
        for (uint32_t spins = 0;; ++spins) {
            v4u v[6];
#pragma unroll
            for (int i = 0; i < 6; ++i) {
                v[i] = v4u{0u, 0u, 0u, 0u};
                if (need >> i & 1)
                    v[i] = __builtin_amdgcn_raw_buffer_load_b128(rs, ((wave + 8 * i) * 64 + lane) * 16, 0, kSC1);
            }
#pragma unroll
            for (int i = 0; i < 6; ++i) {
                if ((need >> i & 1) && v[i].y == tag && v[i].w == tag) {
                    *reinterpret_cast<v2u*>(img + ((wave + 8 * i) * 64 + lane) * 8) = v2u{v[i].x, v[i].z};
                    need &= ~(1u << i);
                }
            }
            if (__builtin_amdgcn_ballot_w64(need != 0) == 0) return true;
            if (spins >= kPollLimit) return false;
            __builtin_amdgcn_s_sleep(1);
        }
    }
    for (uint32_t spins = 0;; ++spins) {
        for (uint32_t i = 0, j = wave; j < nj; ++i, j += 8)
            if (need >> i & 1)
                __builtin_amdgcn_global_load_lds(src + 4 * (j * 64 + lane), (lds_ptr)(stg + j * 1024), 16, 0, kSC1);
        wait_vm();
        for (uint32_t i = 0, j = wave; j < nj; ++i, j += 8) {
            if (need >> i & 1) {
                const v4u v = *reinterpret_cast<const v4u*>(stg + j * 1024 + lane * 16);
                if (v.y == tag && v.w == tag) {
                    *reinterpret_cast<v2u*>(img + (j * 64 + lane) * 8) = v2u{v.x, v.z};
                    need &= ~(1u << i);
                }
            }
        }
        if (__builtin_amdgcn_ballot_w64(need != 0) == 0) return true;
        if (spins >= kPollLimit) return false;
        __builtin_amdgcn_s_sleep(1);
    }
}

// Every wave, after the phase boundary: the activation inputs (the norm weights are already in
// LDS), or the embedding row of the step's token.  A streaming wave's weight loads in flight were
// issued before the boundary, so its wait here costs nothing the next phase would not wait for
// anyway.  Returns false (in the whole wave) if a tagged input did not become current.
__device__ __forceinline__ bool stage_inputs(int kind, const Stage& in, const InputStage& emb, uint32_t K, uint32_t nst,
                                             uint32_t xs_off, uint8_t* lds, uint32_t wave, uint32_t lane) {
    uint8_t* img = lds;
    float* xs = reinterpret_cast<float*>(lds + xs_off);
    bool ok = true;
    if (kind == S_DIGITS) {
        dma_all(in.dig, nst * kStepImg, img, wave, lane);
    } else if (kind == S_TDIGITS) {
        ok = poll_image(in.xt, nst * kStepImg, in.tag, img, img + nst * kStepImg, wave, lane);  // step_xs_offset
    } else if (kind == S_RESID) {
        if (in.xf)
            dma_all(in.xf, K * 4, reinterpret_cast<uint8_t*>(xs), wave, lane);
        else
            ok = poll_tagged(in.xt, K, in.tag, xs, wave * 64 + lane);  // the residual is in xs + K
    } else {
        embed_row(emb, xs, wave * 64 + lane, kThreads);
    }
    wait_vm();
    return ok;
}

// Wave 0: what a residual prologue reads that the phase before it does not change, into its LDS
// slots: the residual (written two phases earlier) and the norm weights.
__device__ __forceinline__ void preload_norms(int kind, const Stage& in, uint32_t K, uint32_t xs_off, uint8_t* lds,
                                              uint32_t lane) {
    float* xs = reinterpret_cast<float*>(lds + xs_off);
    if (kind == S_RESID) dma(in.res, K * 4, reinterpret_cast<uint8_t*>(xs + K), lane);
    if (in.w_a) dma(in.w_a, K * 4, reinterpret_cast<uint8_t*>(xs + 2 * K), lane);
    dma(in.w_n, K * 4, reinterpret_cast<uint8_t*>(xs + 3 * K), lane);
}

// Wave 0 of workgroup 0: the residual left in xs[0, K) by stage_digits.
__device__ __forceinline__ void store_residual(const Stage& in, const uint8_t* lds, uint32_t K, uint32_t xs_off,
                                               uint32_t lane) {
    const v4u* xs = reinterpret_cast<const v4u*>(lds + xs_off);
    for (uint32_t i = lane; i < K / 4; i += 64) {
        const v4u v = xs[i];
        stc16(in.x_out, i * 16, v);
        if (in.snap) stc16(in.snap, i * 16, v);
    }
}

__device__ __forceinline__ void ld8(const float* p, float (&v)[8]) {
    const float4 a = reinterpret_cast<const float4*>(p)[0], b = reinterpret_cast<const float4*>(p)[1];
    v[0] = a.x, v[1] = a.y, v[2] = a.z, v[3] = a.w, v[4] = b.x, v[5] = b.y, v[6] = b.z, v[7] = b.w;
}
__device__ __forceinline__ void st8(float* p, const float (&v)[8]) {
    reinterpret_cast<float4*>(p)[0] = make_float4(v[0], v[1], v[2], v[3]);
    reinterpret_cast<float4*>(p)[1] = make_float4(v[4], v[5], v[6], v[7]);
}

// Digit image of the input before its RMSNorm row factor (K <= 4096, so one octet per thread), all
// threads, from LDS only (16-byte accesses: 8-float strides read element-wise would hit the same
// bank from 16 lanes).  The GEMV input is f32(t rn w_n) with t the residual sum and rn =
// rms(t)^-1; the image holds u = f32(t w_n) instead, and the phase's row sums are scaled by rn
// (norm_factor), so the digits need not wait for the sum of squares of t, whose wave sums this
// leaves in red[8, 16) for norm_factor to add after the caller's barrier.  (The difference is the
// f32 rounding of each input element, about 2^-24 of it.)  The residual sum replaces x in xs[0, K)
// for store_residual.  red: 16 slots.
__device__ __forceinline__ void stage_digits(int kind, const Stage& in, uint32_t K, uint32_t nst, uint32_t xs_off,
                                             uint8_t* lds, double* red) {
    int8_t* dig = reinterpret_cast<int8_t*>(lds);
    BlockTab* tab = reinterpret_cast<BlockTab*>(lds + (size_t)nst * 512);
    float* xs = reinterpret_cast<float*>(lds + xs_off);
    const uint32_t tid = tix(), n8 = K / 8, o = tid;
    const bool ok = o < n8;
    float t[8], v[8], w[8];
#pragma unroll
    for (int k = 0; k < 8; ++k) t[k] = w[k] = 0.0f;
    if (kind == S_EMBED) {
        if (ok) ld8(xs + 8 * o, t);
    } else {
        float x[8], r[8];
#pragma unroll
        for (int k = 0; k < 8; ++k) x[k] = r[k] = 0.0f;
        if (ok) {
            ld8(xs + 8 * o, x);
            ld8(xs + K + 8 * o, r);
            if (in.w_a) ld8(xs + 2 * K + 8 * o, w);
        }
        double ra = 1.0;
        if (in.w_a) {
            double sa = 0.0;
#pragma unroll
            for (int k = 0; k < 8; ++k) sa += (double)x[k] * x[k];
            ra = inv_rms_fast(block_sum_once(sa, red), K, in.eps_a);
        }
#pragma unroll
        for (int k = 0; k < 8; ++k) {
            const float u = in.w_a ? norm_apply(x[k], ra, w[k]) : x[k];
            t[k] = ok ? __fmul_rn(__fadd_rn(u, r[k]), in.scale) : 0.0f;
        }
        if (ok) st8(xs + 8 * o, t);
    }
    double ss = 0.0;
#pragma unroll
    for (int k = 0; k < 8; ++k) ss += (double)t[k] * t[k];
    ss = wave_sum(ss);
    if ((tid & 63) == 0) red[8 + (tid >> 6)] = ss;
    if (ok) ld8(xs + 3 * K + 8 * o, w);
#pragma unroll
    for (int k = 0; k < 8; ++k) v[k] = ok ? __fmul_rn(t[k], w[k]) : 0.0f;
    float m, sum;
    quad_stats(v, m, sum);
    const uint32_t b = o >> 2, p = o & 3;
    if (b < nst * 4) {
        digits8(v, m, dig, b, p);
        if (p == 0) tab[b] = block_tab(m, sum);
    }
}

// The RMSNorm row factor of a residual prologue, from the wave sums stage_digits left in red
// (after a barrier), in block_sum_once's order.
__device__ __forceinline__ double norm_factor(const double* red, uint32_t K, float eps) {
    const double ss = ((red[8] + red[9]) + (red[10] + red[11])) + ((red[12] + red[13]) + (red[14] + red[15]));
    return inv_rms_fast(ss, K, eps);
}

// Digit image words of one 32-element block held by a quad (8 values per lane), stored
// coherently into the image at block b.
__device__ __forceinline__ void quad_digits_store(const float (&v)[8], int8_t* img, uint32_t nst, uint32_t b,
                                                  uint32_t p) {
    float m, sum;
    quad_stats(v, m, sum);
    uint32_t w[4][2];
    digit_words(v, m, w);
#pragma unroll
    for (int t = 0; t < 4; ++t) stc8(img, (b * 4 + t) * 32 + 8 * p, v2u{w[t][0], w[t][1]});
    if (p == 0) {
        const BlockTab e = block_tab(m, sum);
        stc16(img, nst * 512 + b * 16,
              v4u{__float_as_uint(e.s14), __float_as_uint(e.s21), __float_as_uint(e.nbias), 0u});
    }
}

// The same words as tagged pieces (poll_image) of a tagged image.
__device__ __forceinline__ void quad_digits_store_tagged(const float (&v)[8], uint32_t* img, uint32_t nst, uint32_t b,
                                                         uint32_t p, uint32_t tag) {
    float m, sum;
    quad_stats(v, m, sum);
    uint32_t w[4][2];
    digit_words(v, m, w);
#pragma unroll
    for (int t = 0; t < 4; ++t) stc16(img, 2 * ((b * 4 + t) * 32 + 8 * p), v4u{w[t][0], tag, w[t][1], tag});
    if (p == 0) {
        const BlockTab e = block_tab(m, sum);
        stc16(img, 2 * (nst * 512 + b * 16), v4u{__float_as_uint(e.s14), tag, __float_as_uint(e.s21), tag});
        stc16(img, 2 * (nst * 512 + b * 16) + 16, v4u{__float_as_uint(e.nbias), tag, 0u, tag});
    }
}

// ---- attention phase ------------------------------------------------------------------------------

// Work item (KV head h, chunk c) of the visible range runs with all 512 threads; the last chunk
// of a head to finish merges the head's partials and writes the digit image of its query heads'
// outputs for the o-proj GEMV.  Chunks of at most StepArgs::stage_clen tokens have their cached K
// and V rows staged in LDS before the attention phase opens.
template <int GQ>
constexpr uint32_t stage_clen_max() {
    return GQ == 4 ? 32u : 64u;
}

// LDS of an attention item.  The "pre" part (RoPE angles, q/k norm weights, staged K/V rows) is
// written by the streaming waves once they have consumed their qkv records, while wave 0 finishes
// the qkv phase, so it lies clear of everything the qkv phase touches (step_attn_layout: above its
// digit image and clear of the residual it still reads); the "transient" part is written after the
// phase opens, from offset 0.  The merge reuses the space from offset 0: the head's chunk partials,
// then the merged outputs.
template <int GQ>
struct AttnLds {
    static constexpr int D = 256, NH = GQ + 2;
    // transient
    float* nrm;       // [NH][D] q heads, k, v of the new token (raw, then normalised)
    float* qs;        // [GQ][D] rotated queries
    float* scores;    // [GQ][kStepMaxClen]
    float* vred;      // [16][GQ][D]
    double* dred;     // [8][NH] (the q/k/v norms use [NH][2])
    float* fred;      // [8]
    uint16_t* knew;   // [D] new K row (fp16)
    uint16_t* vnew;   // [D] new V row (fp16)
    // pre
    double* rope;     // cos [128], sin [128] of pos * inv_freq (written after the phase opens)
    double* ifreq;    // [128] the layer's RoPE inverse frequencies
    float* qnw;       // [D] q_norm weights
    float* knw;       // [D] k_norm weights
    uint16_t* kst;    // [stage_clen][D] fp16 K rows of the chunk
    uint16_t* vst;    // [stage_clen][D] fp16 V rows
    static constexpr size_t transient_bytes() {
        return 4 * (NH * D + GQ * D + GQ * kStepMaxClen + 16 * GQ * D) + 8 * 8 * NH + 4 * 8 + 2 * 2 * D;
    }
    static constexpr size_t pre_bytes(uint32_t sclen) { return 8 * 384 + 4 * 2 * D + 2 * 2 * (size_t)sclen * D; }
    __device__ AttnLds(uint8_t* lds, uint32_t pre_off, uint32_t sclen) {
        nrm = reinterpret_cast<float*>(lds);
        qs = nrm + NH * D;
        scores = qs + GQ * D;
        vred = scores + GQ * kStepMaxClen;
        dred = reinterpret_cast<double*>(vred + 16 * GQ * D);
        fred = reinterpret_cast<float*>(dred + 8 * NH);
        knew = reinterpret_cast<uint16_t*>(fred + 8);
        vnew = knew + D;
        rope = reinterpret_cast<double*>(lds + pre_off);
        ifreq = rope + 256;
        qnw = reinterpret_cast<float*>(ifreq + 128);
        knw = qnw + D;
        kst = reinterpret_cast<uint16_t*>(knw + D);
        vst = kst + (size_t)sclen * D;
    }
};

// Streaming wave i of n, once it has consumed its qkv records (nothing here depends on this step's
// q, k, v): its share of the RoPE inverse frequencies, the q/k norm weights and the chunk's cached
// K and V rows (two rows per copy instruction, pairs i, i + n, ..), copied into the "pre" LDS
// part.  Issued here rather than by wave 0 during the qkv phase: the copies queue behind the weight
// ring's loads, and wave 0 would wait for them before storing the qkv outputs the attention items
// need.  The caller waits for the copies before the attention phase.
template <int GQ>
__device__ __forceinline__ void attention_pre(CLayer& L, const StepArgs& a, uint32_t pos, uint32_t h, uint32_t c,
                                              uint32_t clen, uint32_t start, uint8_t* lds, uint32_t i, uint32_t n,
                                              uint32_t lane) {
    AttnLds<GQ> m(lds, a.attn_pre_off, a.stage_clen);
    const uint32_t t0 = start + c * clen, t1 = min(pos + 1, t0 + clen);
    if (i == 0) dma(L.inv_freq, 8 * 128, reinterpret_cast<uint8_t*>(m.ifreq), lane);
    if (i == 1 % n) dma(L.q_norm, 4 * 256, reinterpret_cast<uint8_t*>(m.qnw), lane);
    if (i == 2 % n) dma(L.k_norm, 4 * 256, reinterpret_cast<uint8_t*>(m.knw), lane);
    if (clen <= a.stage_clen) {
        const uint32_t old_end = min(t1, pos);  // the new token's row is computed in the phase
        for (uint32_t t = t0 + 2 * i; t < old_end; t += 2 * n) {  // two 512-byte rows per wave instruction
            const uint32_t row = t + (lane >> 5);
            if (row < old_end) {
                const size_t src = ((size_t)h * L.ring + row % L.ring) * 256 + (lane & 31) * 8;
                __builtin_amdgcn_global_load_lds(L.kcache + src, (lds_ptr)(m.kst + (t - t0) * 256), 16, 0, 0);
                __builtin_amdgcn_global_load_lds(L.vcache + src, (lds_ptr)(m.vst + (t - t0) * 256), 16, 0, 0);
            }
        }
    }
}

// Streaming wave 1 (the one that copied the RoPE inverse frequencies in attention_pre), after its
// copies are waited for: the RoPE angles of this position into the pre part.  The item reads them
// after its first barrier, which the streaming waves reach only after this.
template <int GQ>
__device__ __forceinline__ void attention_rope(const StepArgs& a, uint32_t pos, uint8_t* lds, uint32_t lane) {
    AttnLds<GQ> m(lds, a.attn_pre_off, a.stage_clen);
#pragma unroll
    for (int i = 0; i < 2; ++i) {
        const uint32_t f = lane + 64 * i;
        double sn, cs;
        sincos((double)pos * m.ifreq[f], &sn, &cs);
        m.rope[f] = cs;
        m.rope[128 + f] = sn;
    }
}

// One attention item.  Wave 0 does the item's global accesses (the streaming waves' weight loads
// stay in flight), except for chunks too long to stage, whose K/V rows every wave reads directly,
// and the merge's copy of the chunk partials.  Barriers: staged; norms summed; q/k rotated;
// scores; softmax; values; partial; published (and, merging: partials copied; outputs merged).
template <int GQ, bool XL>
__device__ __forceinline__ void attention_item(CLayer& L, const StepArgs& a, uint32_t pos, uint32_t h, uint32_t c,
                                               uint32_t chunks, uint32_t cmax, uint32_t clen, uint32_t start,
                                               uint32_t tag, uint8_t* lds, int* flag, int* bad, const Grid& g) {
    constexpr int D = 256, NH = GQ + 2;
    // XCD-local layout: this head group's q/k/v and chunk partials were written by workgroups of
    // this XCD, so they are read from its L2 (non-temporal loads: they miss the CU's L1, where a
    // poll would otherwise keep hitting a stale line) and the merge ticket is an L2 atomic
    constexpr int kPol = XL ? kNT : kSC1;
    constexpr int kSt = XL ? kSC0 : kSC1;  // stores: into the XCD's L2, or through to the memory side
    constexpr int kScope = XL ? __HIP_MEMORY_SCOPE_WORKGROUP : __HIP_MEMORY_SCOPE_AGENT;
    AttnLds<GQ> sh(lds, a.attn_pre_off, a.stage_clen);
    float* nrm = sh.nrm;
    float* qs = sh.qs;
    float* scores = sh.scores;
    float* vred = sh.vred;
    double* dred = sh.dred;
    float* ml = sh.fred;  // [GQ][2]: max and sum of each query head's softmax

    const uint32_t tid = tix(), lane = tid & 63, wave = wave_id();
    const uint32_t t0 = start + c * clen, t1 = min(pos + 1, t0 + clen), n = t1 - t0;
    const uint32_t ring = L.ring;
    const bool append = t1 == pos + 1;
    const bool staged = clen <= a.stage_clen;
    const int nh = append ? NH : GQ;  // heads normalised here: the queries, and k, v of the new token

    // This token's query heads (and k, v when the chunk ends at it), computed by the qkv phase and
    // handed over as (value, tag) pairs (poll_tagged): 16-byte piece p (two values) of the item
    // is copied to vred + 16 p, and re-copied until both its tags are current; nrm[2 p, 2 p + 2)
    // then takes its values.  Piece j 64 + lane of copy instruction j.
    if (wave == 0) {
        constexpr int J = 2 * NH;  // copy instructions for every head (D / 2 pieces = 2 x 64 each)
        const uint32_t P = (uint32_t)nh * (D / 2);
        uint8_t* stg = reinterpret_cast<uint8_t*>(vred);
        auto src = [&](int j) -> const uint32_t* {  // element of piece j 64 + lane
            const uint32_t p = (uint32_t)j * 64 + lane, q = p / (D / 2), e = 2 * (p % (D / 2));
            const uint32_t base = q < GQ ? (h * GQ + q) * D : (q == GQ ? L.qn : L.v_off) + h * D;
            return a.QKVT + 2 * (size_t)(base + e);
        };
        uint32_t need = 0;
#pragma unroll
        for (int j = 0; j < J; ++j)
            if ((uint32_t)j * 64 + lane < P) need |= 1u << j;
        bool ok = true;
        for (uint32_t spins = 0;; ++spins) {
#pragma unroll
            for (int j = 0; j < J; ++j)
                if (need >> j & 1)
                    __builtin_amdgcn_global_load_lds(src(j), (lds_ptr)(stg + j * 1024), 16, 0, kPol);
            wait_vm();
#pragma unroll
            for (int j = 0; j < J; ++j) {
                if (need >> j & 1) {
                    const v4u v = *reinterpret_cast<const v4u*>(stg + j * 1024 + lane * 16);
                    if (v.y == tag && v.w == tag) {
                        reinterpret_cast<v2u*>(nrm)[j * 64 + lane] = v2u{v.x, v.z};
                        need &= ~(1u << j);
                    }
                }
            }
            if (__builtin_amdgcn_ballot_w64(need != 0) == 0) break;
            if (spins >= kPollLimit) {
                ok = false;
                break;
            }
            __builtin_amdgcn_s_sleep(1);
        }
        if (!ok) *bad = 1;
    }
    __syncthreads();
    if (__builtin_amdgcn_readfirstlane(*bad)) return;
    stamp(g, M_STAGED);

    // RMSNorm of each head over its 256 channels, then NeoX RoPE on the pairs (i, i + 128): head q
    // runs on waves 2 (q % 4) and 2 (q % 4) + 1, whose lane l holds both channels of pair l (even
    // wave) or 64 + l (odd wave), so a head's sum of squares is its two waves' sums, added in pair
    // order, and the rotation needs no exchange.  Heads q and q + 4 share waves (GQ = 4).
    const uint32_t pi = tid & (D / 2 - 1);
    for (uint32_t q = tid >> 7; q < (uint32_t)nh; q += 4) {  // wave-uniform
        const float x0 = nrm[q * D + pi], x1 = nrm[q * D + pi + D / 2];
        const double v = wave_sum((double)x0 * (double)x0 + (double)x1 * (double)x1);
        if (lane == 0) dred[2 * q + (wave & 1)] = v;
    }
    __syncthreads();
    {
        const double cs = sh.rope[pi], sn = sh.rope[128 + pi];
        for (uint32_t q = tid >> 7; q < (uint32_t)nh; q += 4) {
            const float x0 = nrm[q * D + pi], x1 = nrm[q * D + pi + D / 2];
            const double ss = dred[2 * q] + dred[2 * q + 1];
            float y0, y1;
            if (q < GQ) {
                const double r = inv_rms_fast(ss, D, L.q_eps);
                y0 = norm_apply(x0, r, sh.qnw[pi]);
                y1 = norm_apply(x1, r, sh.qnw[pi + D / 2]);
            } else if (q == GQ) {
                const double r = inv_rms_fast(ss, D, L.k_eps);
                y0 = norm_apply(x0, r, sh.knw[pi]);
                y1 = norm_apply(x1, r, sh.knw[pi + D / 2]);
            } else {
                const double r = L.v_norm ? inv_rms_fast(ss, D, L.v_eps) : 1.0;
                y0 = L.v_norm ? (float)__dmul_rn((double)x0, r) : x0;
                y1 = L.v_norm ? (float)__dmul_rn((double)x1, r) : x1;
                const uint16_t v0 = f2h(y0), v1 = f2h(y1);
                sh.vnew[pi] = v0;
                sh.vnew[pi + D / 2] = v1;
                if (staged) {
                    sh.vst[(pos - t0) * D + pi] = v0;
                    sh.vst[(pos - t0) * D + pi + D / 2] = v1;
                }
                continue;
            }
            const double u = (double)y0, w = (double)y1;
            const float r0 = (float)__dsub_rn(__dmul_rn(u, cs), __dmul_rn(w, sn));
            const float r1 = (float)__dadd_rn(__dmul_rn(u, sn), __dmul_rn(w, cs));
            if (q < GQ) {
                qs[q * D + pi] = r0;
                qs[q * D + pi + D / 2] = r1;
            } else {
                const uint16_t k0 = f2h(r0), k1 = f2h(r1);
                sh.knew[pi] = k0;
                sh.knew[pi + D / 2] = k1;
                if (staged) {
                    sh.kst[(pos - t0) * D + pi] = k0;
                    sh.kst[(pos - t0) * D + pi + D / 2] = k1;
                }
            }
        }
    }
    __syncthreads();

    // scores: 16 lanes per token (16 channels each), 32 token groups; q is re-read from LDS for
    // every token (registers stay free for the weight loads in flight)
    // The K and V rows come from LDS (staged chunk, or the new token) or from the cache; the two
    // kinds of chunk run separate loops, so a staged chunk's loops hold no global load, and the
    // compiler has no reason to wait for a streaming wave's weight loads in flight.
    auto score_rows = [&](auto staged_c) {
        constexpr bool ST = decltype(staged_c)::value;
        const uint32_t grp = tid >> 4, j = tid & 15;
        for (uint32_t t = t0 + grp; t < t1; t += 32) {
            v4u k0, k1;
            if (ST || t == pos) {
                const uint16_t* kr = ST ? sh.kst + (t - t0) * D : sh.knew;
                const v4u* kp = reinterpret_cast<const v4u*>(kr + 16 * j);
                k0 = kp[0];
                k1 = kp[1];
            } else {
                const uint16_t* kp = L.kcache + ((size_t)h * ring + t % ring) * D + 16 * j;
                k0 = *gp(reinterpret_cast<const v4u*>(kp));
                k1 = *gp(reinterpret_cast<const v4u*>(kp + 8));
            }
            const uint32_t kw[8] = {k0.x, k0.y, k0.z, k0.w, k1.x, k1.y, k1.z, k1.w};
            float kf[16];
#pragma unroll
            for (int e = 0; e < 8; ++e) {
                kf[2 * e] = h2f((uint16_t)(kw[e] & 0xFFFFu));
                kf[2 * e + 1] = h2f((uint16_t)(kw[e] >> 16));
            }
#pragma unroll
            for (int q = 0; q < GQ; ++q) {
                const float4* qp = reinterpret_cast<const float4*>(qs + q * D + 16 * j);
                float d = 0.0f;
#pragma unroll
                for (int e4 = 0; e4 < 4; ++e4) {
                    const float4 qv = qp[e4];
                    d = fmaf(qv.x, kf[4 * e4], d);
                    d = fmaf(qv.y, kf[4 * e4 + 1], d);
                    d = fmaf(qv.z, kf[4 * e4 + 2], d);
                    d = fmaf(qv.w, kf[4 * e4 + 3], d);
                }
                d = row_sum(d);
                if (j == 0) scores[q * kStepMaxClen + (t - t0)] = d * L.scale;
            }
        }
    };
    // scores: 16 lanes per token (16 channels each), 32 token groups; q is re-read from LDS for
    // every token (registers stay free for the weight loads in flight)
    if (staged) score_rows(std::true_type{});
    else score_rows(std::false_type{});
    __syncthreads();

    // softmax: wave q < GQ normalises query head q's scores on its own (no block reduction)
    if (wave < (uint32_t)GQ) {
        float* sc = scores + wave * kStepMaxClen;
        float mx = -INFINITY;
        for (uint32_t i = lane; i < n; i += 64) mx = fmaxf(mx, sc[i]);
        mx = wave_max(mx);
        float sum = 0.0f;
        for (uint32_t i = lane; i < n; i += 64) {
            const float p = expf(sc[i] - mx);
            sc[i] = p;
            sum += p;
        }
        sum = wave_sum(sum);
        if (lane == 0) {
            ml[2 * wave] = mx;
            ml[2 * wave + 1] = sum;
        }
    }
    __syncthreads();

    // values: 32 lanes per token row (8 channels each), 16 token groups
    auto value_rows = [&](auto staged_c) {
        constexpr bool ST = decltype(staged_c)::value;
        const uint32_t tg = tid >> 5, dl = tid & 31;
        float acc[GQ][8];
#pragma unroll
        for (int q = 0; q < GQ; ++q)
#pragma unroll
            for (int e = 0; e < 8; ++e) acc[q][e] = 0.0f;
        for (uint32_t t = t0 + tg; t < t1; t += 16) {
            v4u vv;
            if (ST || t == pos) {
                const uint16_t* vr = ST ? sh.vst + (t - t0) * D : sh.vnew;
                vv = *reinterpret_cast<const v4u*>(vr + 8 * dl);
            } else {
                vv = *gp(reinterpret_cast<const v4u*>(L.vcache + ((size_t)h * ring + t % ring) * D + 8 * dl));
            }
            const uint32_t vw[4] = {vv.x, vv.y, vv.z, vv.w};
            float vf[8];
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                vf[2 * e] = h2f((uint16_t)(vw[e] & 0xFFFFu));
                vf[2 * e + 1] = h2f((uint16_t)(vw[e] >> 16));
            }
#pragma unroll
            for (int q = 0; q < GQ; ++q) {
                const float p = scores[q * kStepMaxClen + (t - t0)];
#pragma unroll
                for (int e = 0; e < 8; ++e) acc[q][e] = fmaf(p, vf[e], acc[q][e]);
            }
        }
#pragma unroll
        for (int q = 0; q < GQ; ++q)
#pragma unroll
            for (int e = 0; e < 8; ++e) vred[(tg * GQ + q) * D + 8 * dl + e] = acc[q][e];
    };
    if (staged) value_rows(std::true_type{});
    else value_rows(std::false_type{});
    __syncthreads();

    // chunk partial o[q][d] (unnormalised), m[q], l[q], staged in LDS and stored by wave 0; a chunk
    // is `stride` floats, GQ (D + 2) rounded up to whole 16-byte pieces
    constexpr uint32_t stride = step_part_stride(GQ);
    static_assert(stride % 4 == 0 && stride >= GQ * (D + 2), "chunk partial stride");
    float* pst = scores;  // [GQ][D + 2]; the scores are no longer needed
    for (uint32_t i = tid; i < GQ * D; i += kThreads) {
        const uint32_t q = i / D, d = i % D;
        float t = 0.0f;
#pragma unroll
        for (int g2 = 0; g2 < 16; ++g2) t += vred[(g2 * GQ + q) * D + d];
        pst[q * (D + 2) + d] = t;
    }
    if (tid < 2 * GQ) pst[(tid >> 1) * (D + 2) + D + (tid & 1)] = ml[tid];
    __syncthreads();
    stamp(g, M_DIGITS);
    float* const head_part = a.part + (size_t)h * cmax * stride;
    if (wave == 0) {
        if (append) {  // the new K/V rows into the cache (this step reads them from LDS)
            const size_t slot = ((size_t)h * ring + pos % ring) * D;
            *gp(reinterpret_cast<v2u*>(L.kcache + slot) + lane) = reinterpret_cast<const v2u*>(sh.knew)[lane];
            *gp(reinterpret_cast<v2u*>(L.vcache + slot) + lane) = reinterpret_cast<const v2u*>(sh.vnew)[lane];
        }
        // stride * 4 bytes per chunk: a multiple of 16, the padding included
        const v4u* ps = reinterpret_cast<const v4u*>(pst);
        for (uint32_t i = lane; i < stride / 4; i += 64) st16p<kSt>(head_part, (c * stride + 4 * i) * 4, ps[i]);
        wait_vm();
        if (lane == 0) {
            const uint32_t ticket =
                __hip_atomic_fetch_add(a.counters + h, 1u, __ATOMIC_RELAXED, kScope);
            *flag = ticket == chunks - 1;
        }
        wait_vm();
    }
    __syncthreads();
    stamp(g, M_STREAMED);
    if (!__builtin_amdgcn_readfirstlane(*flag)) return;

    // merge (last chunk of this head): M = max_c m_c, w_c = exp(m_c - M), output
    // sum_c w_c o_c / sum_c w_c l_c, in chunk order; the weights once per (query head, chunk)
    float* mrg = reinterpret_cast<float*>(lds);  // [chunks][stride]
    float* outv = mrg + chunks * stride;        // [GQ][D]
    float* wts = outv + GQ * D;                 // [GQ][chunks]
    dma_all<kPol>(head_part, chunks * stride * 4, lds, wave, lane);
    wait_vm();
    __syncthreads();
    if (wave < (uint32_t)GQ) {
        float M = -INFINITY;
        for (uint32_t k = lane; k < chunks; k += 64) M = fmaxf(M, mrg[k * stride + wave * (D + 2) + D]);
        M = wave_max(M);
        for (uint32_t k = lane; k < chunks; k += 64) wts[wave * chunks + k] = expf(mrg[k * stride + wave * (D + 2) + D] - M);
    }
    __syncthreads();
    for (uint32_t i = tid; i < GQ * D; i += kThreads) {
        const uint32_t q = i / D, d = i % D;
        float Lq = 0.0f, acc = 0.0f;
        for (uint32_t k = 0; k < chunks; ++k) {
            const float* pk = mrg + k * stride + q * (D + 2);
            const float w = wts[q * chunks + k];
            Lq = fmaf(w, pk[D + 1], Lq);
            acc = fmaf(w, pk[d], acc);
        }
        outv[i] = acc / Lq;
    }
    __syncthreads();
    // digit image blocks (h GQ + q) * 8 + b of the o-proj input: 4 lanes of wave 0 per block
    const uint32_t nst_att = L.o.nst;
    if (wave == 0) {
        for (uint32_t base = 0; base < 32 * GQ; base += 64) {
            const uint32_t i = base + lane;
            if (i < 32 * GQ) {
                const uint32_t blk = i >> 2, p = i & 3;
                float v[8];
#pragma unroll
                for (int k = 0; k < 8; ++k) v[k] = outv[blk * 32 + 8 * p + k];
                quad_digits_store_tagged(v, reinterpret_cast<uint32_t*>(a.att_img), nst_att, h * GQ * 8 + blk, p, tag);
            }
        }
        if (lane == 0) __hip_atomic_store(a.counters + h, 0u, __ATOMIC_RELAXED, kScope);
        wait_vm();
    }
}

// ---- the kernel -----------------------------------------------------------------------------------

// Phases of a layer, in order.
enum PhaseKind { P_QKV = 0, P_ATTN, P_OPROJ, P_GATEUP, P_DOWN, kPhases };

// One GEMV phase of a layer, read from the layer table.
struct Gemv {
    Shape sh;
    int in_kind;     // StageKind
    Stage in;
    InputStage emb;  // S_EMBED
    uint32_t K;      // input width
    float* y;        // outputs (qkv, and the last layer's down, read by the head)
    uint32_t* yt;    // outputs as (value, tag) pairs (o-proj, down): the next phase polls them
    uint32_t ytag;
    uint32_t rows;
    uint32_t act_nst;
};

__device__ __forceinline__ Shape shape_of(CQ4View& m, bool pair) {
    Shape sh;
    sh.nst = __builtin_amdgcn_readfirstlane(m.nst);
    sh.T = pair ? 4u : 1u;
    sh.units = __builtin_amdgcn_readfirstlane(pair ? (m.rows + 31) / 32 : (m.rows + 15) / 16);
    return sh;
}

// tag0: the tag of layer 0's handed-over vectors in this launch (layer l: tag0 + l).
__device__ __forceinline__ Gemv describe(const StepArgs& a, uint32_t l, uint32_t kind, uint32_t tag0 = 0) {
    CLayer& L = layer_at(a, l);
    Gemv d{};
    if (kind == P_QKV) {
        d.sh = shape_of(L.qkv, false);
        d.K = a.hidden;
        d.yt = a.QKVT;
        d.ytag = tag0 + l;
        d.rows = L.qkv.rows;
        if (l == 0 && !a.prev_post_ffn) {
            d.in_kind = S_EMBED;
            d.emb.table = a.table;
            d.emb.ids = a.ids;
            d.emb.state = a.state;
            d.emb.emb_scale = a.emb_scale;
        } else if (l == 0) {
            d.in_kind = S_RESID;
            d.in.xf = a.D;
            d.in.res = a.H;
            d.in.w_a = a.prev_post_ffn;
            d.in.eps_a = a.prev_post_ffn_eps;
            d.in.scale = a.prev_scale;
        } else {
            CLayer& P = layer_at(a, l - 1);
            d.in_kind = S_RESID;
            d.in.xt = a.DT;
            d.in.tag = tag0 + l - 1;
            d.in.res = a.H;
            d.in.w_a = P.post_ffn;
            d.in.eps_a = P.post_ffn_eps;
            d.in.scale = P.layer_scale;
            d.in.snap = a.snap ? a.snap + (size_t)(l - 1) * a.hidden : nullptr;
        }
        d.in.w_n = L.input_norm;
        d.in.eps_n = L.input_eps;
        d.in.x_out = a.X;
    } else if (kind == P_OPROJ) {
        d.sh = shape_of(L.o, false);
        d.in_kind = S_TDIGITS;
        d.in.xt = reinterpret_cast<const uint32_t*>(a.att_img);
        d.in.tag = tag0 + l;
        d.K = L.o.blocks * 32;
        d.yt = a.PROJT;
        d.ytag = tag0 + l;
        d.rows = L.o.rows;
    } else if (kind == P_GATEUP) {
        d.sh = shape_of(L.gate, true);
        d.in_kind = S_RESID;
        d.in.xt = a.PROJT;
        d.in.tag = tag0 + l;
        d.in.res = a.X;
        d.in.w_a = L.post_attn;
        d.in.eps_a = L.post_attn_eps;
        d.in.scale = 1.0f;
        d.in.w_n = L.ffn_norm;
        d.in.eps_n = L.ffn_eps;
        d.in.x_out = a.H;
        d.K = a.hidden;
        d.act_nst = L.down.nst;
    } else {
        d.sh = shape_of(L.down, false);
        d.in_kind = S_DIGITS;
        d.in.dig = a.act_img;
        d.K = a.inter;
        if (l + 1 < a.n_layers) {
            d.yt = a.DT;
            d.ytag = tag0 + l;
        } else {
            d.y = a.D;
        }
        d.rows = L.down.rows;
    }
    return d;
}

// Attention work of a layer at position pos: chunks of at least kAttnMinChunk tokens, at most
// StepLayer::chunks_max per KV head (cmax: the chunk partials' stride per KV head); item i runs on
// workgroup grid - 1 - i.
struct AttnGeo {
    uint32_t start, chunks, clen, cmax, items;
};

__device__ __forceinline__ AttnGeo attn_geo(CLayer& L, uint32_t pos, uint32_t cmax) {
    AttnGeo g;
    const uint32_t nvis = L.window ? min(pos + 1, L.window) : pos + 1;
    g.start = pos + 1 - nvis;
    g.cmax = cmax;
    uint32_t chunks = min(L.chunks_max, (nvis + kAttnMinChunk - 1) / kAttnMinChunk);
    g.clen = (nvis + chunks - 1) / chunks;
    g.chunks = (nvis + g.clen - 1) / g.clen;
    g.items = L.kv_heads * g.chunks;
    return g;
}

// The attention item (KV head h, chunk c) of this workgroup, if it has one: item i = h chunks + c
// runs on workgroup grid - 1 - i, or in the XCD-local layout chunk c of head h on workgroup
// 8 (grid / 8 - 1 - c) + h (every chunk of a head on one XCD).
template <bool XL>
__device__ __forceinline__ bool attn_item(const AttnGeo& ag, uint32_t& h, uint32_t& c) {
    if constexpr (XL) {
        const uint32_t b = blockIdx.x;
        h = b % kXcds;
        c = 256u / kXcds - 1 - b / kXcds;  // the XCD-local layout's grid
        return c < ag.chunks && h * ag.chunks < ag.items;
    } else {
        const uint32_t item = gridDim.x - 1 - blockIdx.x;
        h = item / max(ag.chunks, 1u);
        c = item % max(ag.chunks, 1u);
        return item < ag.items;
    }
}

}  // namespace

// Wave 0: copies for phase ph that do not depend on the phase before it (the norm weights of a
// residual prologue; an attention item's copies are the streaming waves', norms_pre_part).  Issued
// only: the caller waits (wave 0 waits for everything at the end of its epilogue).
template <int GQ, bool XL>
__device__ __forceinline__ void phase_pre(const StepArgs& a, int32_t ph, int32_t n_phases, uint32_t pos, uint8_t* lds,
                                          uint32_t lane) {
    if (ph >= n_phases) return;
    const uint32_t l = (uint32_t)ph / kPhases, kind = (uint32_t)ph % kPhases;
    if (kind == P_QKV || kind == P_GATEUP) {
        const Gemv d = describe(a, l, kind);
        preload_norms(d.in_kind, d.in, d.K, a.xs_off, lds, lane);
    }
}

// The copies for phase ph by the streaming waves once their records are consumed: the residual and
// norm weights of a GEMV phase (qkv, gate/up; waves 1-7 each take every 7th KB), or the attention
// item's pre part (attention_pre; the attention phase's pre part always lies clear of the qkv
// phase's LDS, step_attn_layout).  Returns false for other phases (left to phase_pre on wave 0).
template <int GQ, bool XL>
__device__ __forceinline__ bool norms_pre_part(const StepArgs& a, int32_t ph, int32_t n_phases, uint32_t pos,
                                               uint8_t* lds, uint32_t wave, uint32_t lane) {
    if (ph >= n_phases) return false;
    const uint32_t l = (uint32_t)ph / kPhases, kind = (uint32_t)ph % kPhases;
    if (kind == P_ATTN) {
        CLayer& L = layer_at(a, l);
        const AttnGeo ag = attn_geo(L, pos, a.cmax);
        uint32_t h, c;
        if (attn_item<XL>(ag, h, c))
            attention_pre<GQ>(L, a, pos, h, c, ag.clen, ag.start, lds, wave - 1, kStreamWaves, lane);
        return true;
    }
    if (kind != P_QKV && kind != P_GATEUP) return false;
    const Gemv d = describe(a, l, kind);
    float* xs = reinterpret_cast<float*>(lds + a.xs_off);
    if (d.in_kind == S_RESID)
        dma_part(d.in.res, d.K * 4, reinterpret_cast<uint8_t*>(xs + d.K), wave - 1, kStreamWaves, lane);
    if (d.in.w_a) dma_part(d.in.w_a, d.K * 4, reinterpret_cast<uint8_t*>(xs + 2 * d.K), wave - 1, kStreamWaves, lane);
    dma_part(d.in.w_n, d.K * 4, reinterpret_cast<uint8_t*>(xs + 3 * d.K), wave - 1, kStreamWaves, lane);
    return true;
}

// Lowest LDS byte phase_pre writes for phase ph (no write: ~0).
template <int GQ>
__device__ __forceinline__ size_t phase_pre_low(const StepArgs& a, int32_t ph, int32_t n_phases) {
    if (ph >= n_phases) return ~(size_t)0;
    const uint32_t l = (uint32_t)ph / kPhases, kind = (uint32_t)ph % kPhases;
    if (kind == P_ATTN) return a.attn_pre_off;
    if (kind == P_QKV || kind == P_GATEUP) {
        const Gemv d = describe(a, l, kind);
        return (size_t)a.xs_off + (size_t)4 * d.K;  // from the residual's slot
    }
    return ~(size_t)0;
}

// Wave roles.  Inside a phase, waves 1-7 issue no vector memory instruction but their weight
// loads: the compiler then waits for exactly the ring slot being consumed.  Wave 0 does every
// other global access of the phase (barrier, pre-copies, stores), and every wave-0 block that
// issues one waits for it before the block ends.  A GEMV phase: its boundary (grid barrier or
// tagged input); all waves stage the inputs; all build the digit image from LDS; waves 1-7
// consume their weight stream (refilling the ring with the next phase's records) while wave 0
// stores the residual and prepares the next phase when its LDS is free; wave 0 stores the
// outputs.  Every phase's code appears once in the loop over (layer, phase).
template <int GQ, bool XL>
__global__ __launch_bounds__(512) void decode_step_kernel(StepArgs a) {
    extern __shared__ __align__(16) uint8_t lds[];
    __shared__ float part[kPart];
    __shared__ double red[16];
    __shared__ int ok_flag, att_flag, poll_bad;
    __shared__ uint32_t done_cnt;  // streaming waves done with a GEMV phase, 64 per wave
    __shared__ float act_l[kMaxUnits][32];
    __shared__ __align__(16) uint8_t pf_sink[1024];  // prefetch_records' destination, never read

    if (a.state[ST_STOP]) return;  // uniform: written only before the launch
    const uint32_t tid = threadIdx.x, lane = tid & 63, wave = wave_id();
    // the XCD-local layout runs on exactly 256 workgroups (setup_step): a constant then
    const uint32_t grid = XL ? 256u : gridDim.x;
    const uint32_t pos = a.state[ST_POS];
    const uint32_t tag0 = a.state[ST_EPOCH] * a.tag_stride + 1u + a.tag_base;  // never 0, a cleared pair's tag
    Grid g{a.bar, 0u, 0u, &ok_flag, a.clock};
    stamp(g, M_START);
    bool failed = false;
    const int32_t n_phases = (int32_t)(kPhases * a.n_layers);
    __shared__ uint4 zero_blk[2];
    if (tid < 2) zero_blk[tid] = make_uint4(0u, 0u, 0u, 0u);  // read after the first __syncthreads
    if (tid == 0) done_cnt = 0;
    if (tid == 0) poll_bad = 0;
    Ring r;
    if (wave != 0) {
        const uint32_t w = blockIdx.x * kStreamWaves + (wave - 1);
        const uint64_t o0 = a.stream_off[2 * w], o1 = a.stream_off[2 * w + 1];
        const uint64_t base = reinterpret_cast<uint64_t>(a.stream) + o0;
        r.base_lo = (uint32_t)base;
        r.base_hi = (uint32_t)(base >> 32);
        r.len = (uint32_t)(o1 - o0);
        r.soff = 0;
        r.slot = 0;
        const __amdgpu_buffer_rsrc_t rs = ring_rsrc(r);
#pragma unroll
        for (int u = 0; u < kRing; ++u) ring_fill(r, rs, u, lane);
    } else {
        phase_pre<GQ, XL>(a, 0, n_phases, pos, lds, lane);
        wait_vm();
    }

    for (int32_t ph = 0; ph < n_phases; ++ph) {
        const uint32_t tid = tix(), lane = tid & 63;
        const LaneK lk = lane_k(lane);
        const uint32_t l = (uint32_t)ph / kPhases, kind = (uint32_t)ph % kPhases;
        // The inputs of attention (qkv's outputs), o-proj (the attention image), gate/up (o-proj's
        // outputs) and qkv after layer 0 (down's outputs) are handed over by tags; down opens with a
        // grid barrier.  After a GEMV phase wave 0 has waited for the streaming waves (done_cnt)
        // and for its stores.
        const bool tagged = kind != P_DOWN;
        if (ph > 0) {
            if (tagged) {
                tagged_boundary(g);
            } else if (!grid_sync(g, (uint32_t)(ph - 1) % kPhases == P_ATTN, (uint32_t)ph == a.fail_phase ? 1u : 0u)) {
                failed = true;
                break;
            }
        }
        if (kind == P_ATTN) {
            CLayer& L = layer_at(a, l);
            const AttnGeo ag = attn_geo(L, pos, a.cmax);
            uint32_t h, c;
            if (attn_item<XL>(ag, h, c))
                attention_item<GQ, XL>(L, a, pos, h, c, ag.chunks, ag.cmax, ag.clen, ag.start, tag0 + l, lds, &att_flag,
                                       &poll_bad, g);
            else if (wave != 0)
                prefetch_records(r, pf_sink, lane);
            // the barrier's workgroup fence waits for every LDS write of the workgroup, so the
            // prefetch's DMAs (into pf_sink) complete here, before the o-proj stage
            __syncthreads();
            if (__builtin_amdgcn_readfirstlane(poll_bad)) {
                failed = true;
                break;
            }
            stamp(g, M_STORED);
        } else {
            const Gemv d = describe(a, l, kind, tag0);
            const uint32_t nst = d.sh.nst;
            if (!stage_inputs(d.in_kind, d.in, d.emb, d.K, nst, a.xs_off, lds, wave, lane)) poll_bad = 1;
            __syncthreads();
            if (__builtin_amdgcn_readfirstlane(poll_bad)) {
                failed = true;
                break;
            }
            stamp(g, M_STAGED);
            zero_part_lds(part, tid);
            if (d.in_kind < S_DIGITS) stage_digits(d.in_kind, d.in, d.K, nst, a.xs_off, lds, red);
            __syncthreads();
            stamp(g, M_DIGITS);
            // the next phase's LDS writes may start now if they stay above this phase's image
            const bool pre_now = phase_pre_low<GQ>(a, ph + 1, n_phases) >= (size_t)nst * kStepImg;
            // Each role's code up to its last global access of the phase is one branch, so the
            // compiler's wait model never mixes wave 0's copies into the streaming waves'.
            if (wave != 0) {
                const uint32_t fe = step_units(d.sh.units, blockIdx.x, grid) * d.sh.T * nst;
                consume_phase(r, nst, d.sh.T, __builtin_amdgcn_readfirstlane(fe), lds,
                              reinterpret_cast<const v4i*>(zero_blk), part, wave, lane, lk, &done_cnt);
                // waited for here, so that no LDS copy is pending at the loop's back edge: the
                // compiler would otherwise wait for every load in flight (this wave's weight ring
                // included) before the next phase's first LDS read
                if (pre_now || kind == P_QKV) norms_pre_part<GQ, XL>(a, ph + 1, n_phases, pos, lds, wave, lane);
                wait_vm();
                // the ring's next record into slot 0 now, while the wave waits for the next phase's
                // inputs, rather than at that phase's start, where the moves would delay its first fold
                ring_rotate(r);
                r.slot = 0;
                if (wave == 1 && kind == P_QKV && ph + 1 < n_phases) {  // next: this layer's attention
                    CLayer& L = layer_at(a, l);
                    const AttnGeo ag = attn_geo(L, pos, a.cmax);
                    uint32_t h, c;
                    if (attn_item<XL>(ag, h, c)) attention_rope<GQ>(a, pos, lds, lane);
                }
                if (wave == 1) stamp_at(g, g.p, M_CONSUMED);
            } else {
                // waited for before the outputs are stored: a phase that reads the residual may be
                // ordered after this one only through the outputs' tags
                if (blockIdx.x == 0 && d.in_kind < S_DIGITS) {
                    store_residual(d.in, lds, d.K, a.xs_off, lane);
                    wait_vm();
                }
                stamp(g, M_PRE);
                // the streaming waves with records (wave - 1 < fe) have left their partials in part
                const uint32_t fe = step_units(d.sh.units, blockIdx.x, grid) * d.sh.T * nst;
                // a residual prologue's row factor (1 for an input given as a digit image), while the
                // streaming waves consume: the wave sums it adds are in red since the digits barrier
                const double rn = d.in_kind < S_DIGITS ? norm_factor(red, d.K, d.in.eps_n) : 1.0;
                const uint32_t want = 64u * min(kStreamWaves, fe);
                while (__hip_atomic_load(&done_cnt, __ATOMIC_ACQUIRE, __HIP_MEMORY_SCOPE_WORKGROUP) < want)
                    __builtin_amdgcn_s_sleep(1);
                done_cnt = 0;  // next incremented after the next phase's stage barrier
                stamp(g, M_STREAMED);
                if (!pre_now) phase_pre<GQ, XL>(a, ph + 1, n_phases, pos, lds, lane);
                const uint32_t mu = step_units(d.sh.units, blockIdx.x, grid);
                if (d.y || d.yt) {
                    if (tid < 16 * mu) {
                        const uint32_t k = tid >> 4, rr = tid & 15;
                        uint32_t tile = blockIdx.x + k * grid;
                        if (XL && kind == P_QKV) {
                            CLayer& L = layer_at(a, l);
                            tile = step_qkv_tile(blockIdx.x, k, grid, 1u, L.qn / 16, L.kn / 16);
                        }
                        const uint32_t row = tile * 16 + rr;
                        const float y = (float)(rn * (double)part_sum(part, k, 0, rr));
                        if (row < d.rows) {
                            if (XL && kind == P_QKV)  // read by this XCD's attention items, from its L2
                                st8p<kSC0>(d.yt, row * 8, v2u{__float_as_uint(y), d.ytag});
                            else if (d.yt)
                                stc8(d.yt, row * 8, v2u{__float_as_uint(y), d.ytag});
                            else
                                stc(d.y, row * 4, __float_as_uint(y));
                        }
                    }
                } else {
                    if (tid < 32 * mu) {
                        const uint32_t k = tid >> 5, rr = tid & 31, t = rr >> 4, r16 = rr & 15;
                        const float gt = (float)(rn * (double)part_sum(part, k, t, r16));
                        const float up = (float)(rn * (double)part_sum(part, k, 2 + t, r16));
                        act_l[k][rr] = gelu_mul(gt, up);
                    }
                    __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");  // act_l: written and read by wave 0
                    if (tid < 4 * mu) {
                        const uint32_t k = tid >> 2, p = tid & 3;
                        float v[8];
#pragma unroll
                        for (int e = 0; e < 8; ++e) v[e] = act_l[k][8 * p + e];
                        quad_digits_store(v, a.act_img, d.act_nst, blockIdx.x + k * grid, p);
                    }
                }
                wait_vm();
                stamp(g, M_STORED);
            }
        }
    }
    grid_exit(g, a.state, a.advance != 0, failed);
}

// One workgroup per (workgroup b, streaming wave w) of the step grid, block b * 7 + w - 1: copies
// that wave's records, every GEMV phase of every layer in consume order, from the layers' tiled
// matrices into its run (a unit past the last row tile reads as zero weights).
__global__ __launch_bounds__(256) void stream_repack_kernel(const StepLayer* layers, uint32_t n_layers, uint32_t grid,
                                                            uint32_t xl, uint8_t* stream, const uint64_t* off) {
    const uint32_t b = blockIdx.x / kStreamWaves, w = blockIdx.x % kStreamWaves + 1;
    uint4* dst = reinterpret_cast<uint4*>(stream + off[blockIdx.x]);
    constexpr uint32_t kChunks = kStepRecord / 16;  // 64 code chunks, then 8 scale chunks
    constexpr uint32_t kPer = 256 / kChunks;        // records per pass
    for (uint32_t l = 0; l < n_layers; ++l) {
        const StepLayer& L = layers[l];
        for (uint32_t kind = 0; kind < 4; ++kind) {
            const Q4View& m0 = kind == 0 ? L.qkv : kind == 1 ? L.o : kind == 2 ? L.gate : L.down;
            const bool pair = kind == 2;
            const uint32_t nst = m0.nst, T = pair ? 4u : 1u, tiles = (m0.rows + 15) / 16;
            const uint32_t units = pair ? (m0.rows + 31) / 32 : tiles;
            const uint32_t n = step_wave_records(units, T, nst, b, grid, w);
            for (uint32_t j0 = 0; j0 < n; j0 += kPer) {
                const uint32_t j = j0 + threadIdx.x / kChunks, c = threadIdx.x % kChunks;
                if (threadIdx.x < kPer * kChunks && j < n) {
                    const uint32_t f = w - 1 + kStreamWaves * j, seg = f / nst, st = f % nst, ts = seg % T, k = seg / T;
                    const uint32_t u = b + k * grid;
                    const Q4View& m = pair && ts >= 2 ? L.up : m0;
                    const uint32_t tile = pair ? 2 * u + (ts & 1)
                                               : kind == 0 ? step_qkv_tile(b, k, grid, xl, L.qn / 16, L.kn / 16) : u;
                    const size_t src = (size_t)tile * nst + st;
                    uint4 v = make_uint4(0u, 0u, 0u, 0u);
                    if (tile < tiles)
                        v = c < 64 ? reinterpret_cast<const uint4*>(m.codes)[src * 64 + c]
                                   : reinterpret_cast<const uint4*>(m.scales)[src * 8 + (c - 64)];
                    dst[(size_t)j * kChunks + c] = v;
                }
            }
            dst += (size_t)n * kChunks;
        }
    }
}

hipError_t launch_stream_repack(const StepLayer* layers, uint32_t n_layers, uint32_t grid, uint32_t xcd_local,
                                uint8_t* stream, const uint64_t* stream_off, hipStream_t s) {
    hipLaunchKernelGGL(stream_repack_kernel, dim3(grid * kStreamWaves), dim3(256), 0, s, layers, n_layers, grid,
                       xcd_local, stream, stream_off);
    return hipGetLastError();
}

// Thread 0 of workgroup b stores the XCD it runs on (the XCC_ID hardware register, bits [3:0]).
__global__ __launch_bounds__(64) void xcd_map_kernel(uint32_t* xcc) {
    if (threadIdx.x == 0) xcc[blockIdx.x] = __builtin_amdgcn_s_getreg((15 << 11) | (0 << 6) | 20) & 0xFu;
}

hipError_t step_xcd_map(uint32_t grid, uint32_t* xcc, hipStream_t s) {
    hipLaunchKernelGGL(xcd_map_kernel, dim3(grid), dim3(64), 0, s, xcc);
    return hipGetLastError();
}

uint32_t step_merge_chunks(uint32_t group, size_t lds) {
    // per chunk: its partials and one weight per query head
    const size_t out = (size_t)group * 256 * 4, per = ((size_t)step_part_stride(group) + group) * 4;
    return lds > out ? (uint32_t)((lds - out) / per) : 0u;
}

uint32_t step_xs_offset(uint32_t hidden, uint32_t inter, uint32_t q_dim) {
    const uint32_t nst = std::max({(hidden + 127) / 128, (inter + 127) / 128, (q_dim + 127) / 128});
    // the o-proj image and, above it, the staging of its tagged pieces (poll_image: 1 KB per 64)
    const uint32_t o_img = (q_dim + 127) / 128 * kStepImg, o_stage = (o_img / 8 + 63) / 64 * 1024;
    return (std::max(nst * kStepImg, o_img + o_stage) + 15) / 16 * 16;  // the largest digit image of any GEMV phase
}

// An attention item's LDS.  Its transient part lies at offset 0 (fixed: with a run-time offset the
// compiler cannot keep its addresses apart from the pre part's, and the item ran 0.6 us slower).
// Its pre part is copied while the qkv phase still reads its digit image [0, img) and (workgroup
// 0, store_residual) the residual at [xs, xs + 4 hidden): it goes above the transient part and clear
// of the residual, with as many staged tokens (up to stage_clen_max) as the LDS budget leaves.
// Config 4: pre part at 84480 (above the residual), 64 tokens, 155136 bytes.  Returns the dynamic
// LDS bytes the launch needs.
constexpr size_t kStepLdsBudget = 160 * 1024 - 8 * 1024;  // the CU's LDS less the kernel's static LDS

template <int GQ>
static size_t attn_layout(uint32_t hidden, uint32_t inter, uint32_t q_dim, uint32_t* pre_off, uint32_t* sclen) {
    const size_t xs = step_xs_offset(hidden, inter, q_dim);
    const size_t xs_end = xs + (size_t)4 * hidden * 4;  // x, res, two norm weight vectors
    const size_t res_end = xs + (size_t)4 * hidden;
    const size_t fixed = AttnLds<GQ>::pre_bytes(0), row = AttnLds<GQ>::pre_bytes(1) - fixed;
    size_t p = (AttnLds<GQ>::transient_bytes() + 255) / 256 * 256;
    if (p < res_end && p + AttnLds<GQ>::pre_bytes(stage_clen_max<GQ>()) > xs) p = (res_end + 255) / 256 * 256;
    const size_t fit = kStepLdsBudget > p + fixed ? (kStepLdsBudget - p - fixed) / row : 0;
    *pre_off = (uint32_t)p;
    *sclen = (uint32_t)std::min<size_t>(stage_clen_max<GQ>(), fit);
    return std::max(xs_end, p + AttnLds<GQ>::pre_bytes(*sclen));
}

void step_attn_layout(uint32_t hidden, uint32_t inter, uint32_t q_dim, uint32_t group, uint32_t* pre_off,
                      uint32_t* stage_clen) {
    if (group == 1) (void)attn_layout<1>(hidden, inter, q_dim, pre_off, stage_clen);
    else if (group == 2) (void)attn_layout<2>(hidden, inter, q_dim, pre_off, stage_clen);
    else (void)attn_layout<4>(hidden, inter, q_dim, pre_off, stage_clen);
}

size_t step_lds_bytes(uint32_t hidden, uint32_t inter, uint32_t q_dim, uint32_t group) {
    uint32_t pre_off = 0, sclen = 0;
    return group == 1   ? attn_layout<1>(hidden, inter, q_dim, &pre_off, &sclen)
           : group == 2 ? attn_layout<2>(hidden, inter, q_dim, &pre_off, &sclen)
                        : attn_layout<4>(hidden, inter, q_dim, &pre_off, &sclen);
}

// A plain launch: the grid is the occupancy API's co-resident maximum (step_max_grid, one
// workgroup per CU), so every workgroup of the grid barriers is resident; a grid that were not
// would end in the barriers' spin limit, reported as a failed step, not in a hang.  The
// cooperative launch API gives the same residency and costs about 12 us more per launch.
hipError_t launch_step(const StepArgs& a, uint32_t group, uint32_t grid, size_t lds, hipStream_t s) {
    // the XCD-local instance is compiled for its 256-workgroup grid (setup_step checks both)
    if (a.xcd_local && (group != 2 || grid != 256)) return hipErrorInvalidValue;
    switch (group) {
        case 1: hipLaunchKernelGGL((decode_step_kernel<1, false>), dim3(grid), dim3(kThreads), lds, s, a); break;
        case 2:
            if (a.xcd_local) hipLaunchKernelGGL((decode_step_kernel<2, true>), dim3(grid), dim3(kThreads), lds, s, a);
            else hipLaunchKernelGGL((decode_step_kernel<2, false>), dim3(grid), dim3(kThreads), lds, s, a);
            break;
        case 4: hipLaunchKernelGGL((decode_step_kernel<4, false>), dim3(grid), dim3(kThreads), lds, s, a); break;
        default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

hipError_t step_max_grid(uint32_t group, size_t lds, uint32_t* grid) {
    int dev = 0, cus = 0, per = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e == hipSuccess) e = hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev);
    const void* k = group == 1   ? (const void*)decode_step_kernel<1, false>
                    : group == 2 ? (const void*)decode_step_kernel<2, false>
                                 : (const void*)decode_step_kernel<4, false>;
    if (e == hipSuccess) e = hipOccupancyMaxActiveBlocksPerMultiprocessor(&per, k, kThreads, lds);
    if (e != hipSuccess) return e;
    *grid = per >= 1 ? (uint32_t)(cus / 8 * 8) : 0u;
    return hipSuccess;
}

}  // namespace af
