// wavefront.hip.h -- the stripe-pipeline machinery shared by every soft-DP sweep
// (linear / affine Smith-Waterman, DTW; value, marginal, tangent and dual sweeps).
//
// Geometry (one workgroup per batch element, NW wave64s):
//   * DP rows are cut into 64-row stripes; stripe s runs on wave s % NW.  Lane r
//     holds DP row 64*s + r + 1 and sweeps the columns with a one-column skew per
//     lane: at step t lane r works on column t - r (0-based), so the wave's 64 cells
//     of one step lie on one anti-diagonal and a stripe takes L2 + 63 steps;
//   * neighbours inside a stripe move between lanes with DPP; the stripe boundary
//     goes through an LDS ring (one slot per column) from the producing stripe's
//     edge lane to the consuming stripe's edge lane;
//   * waves never meet at a barrier.  Each wave publishes its progress word
//     (stripe * PROG_STRIDE + chunks done) in LDS; a stripe waits, chunk by chunk,
//     for the part of the neighbouring stripe it reads and, so that a ring is not
//     overwritten, for its consumer to have caught up.  Every wait is bounded: a
//     wave that polls SPIN_LIMIT times sets bit 0 of the element's status word and
//     goes on, so a logic error can never hang the GPU;
//   * per-cell inputs (scores, costs, tangents) arrive one chunk (P steps) ahead by
//     direct-to-LDS loads, laid out so the per-step column read is conflict-free;
//     stored DP tables use a skewed layout table[stripe][step][lane] (one 256-byte
//     row per wave step) that both sweep directions stream contiguously.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "dp_common.hip.h"

namespace d2p_amd {
namespace wf {

constexpr int NW = 8;                 // waves per workgroup
constexpr int SPIN_LIMIT = 1 << 22;   // default polls before a wait gives up (~0.2 s in LDS)
constexpr int PROG_STRIDE = 1 << 16;  // progress word = stripe * PROG_STRIDE + chunks done
constexpr int APAD = 18;              // table steps stored before step 0 (>= P + 2)
constexpr int STEP_QUANTUM = 16;      // stored steps are a multiple of this (>= every P)
constexpr size_t TRASH_BYTES = 256;   // one line that masked lanes store into

// Shape limits of the pipeline beyond the reference's (L1 + 1) * (L2 + 1) <= INT32_MAX:
// progress words count a stripe's chunks in 16 bits (P >= 4 steps per chunk, so
// max_L2 + 63 < 2^18) and its stripe in the high half of an int (< 32768 stripes).
// Per-lane matrix offsets are taken from the stripe's first row, so they span at
// most 64 rows and set no limit of their own.
constexpr int MAX_L2 = (1 << 18) - 64;
constexpr int MAX_L1 = 32767 * 64;

__host__ inline bool table_fits_int32(int max_L1, int max_L2) {
    return ((long long)max_L1 + 1) * ((long long)max_L2 + 1) <= 2147483647LL;
}

// A stripe's chunk k reads boundary values the neighbouring stripe produces up to
// 62 + P steps later in its own sweep, i.e. in its chunk k + 1 + 62/P; so it waits
// until that stripe has completed k + lead(P) chunks.
__host__ __device__ constexpr int lead(int P) { return 2 + 62 / P; }

// Ring length (columns) of one stripe boundary.  It must exceed the pipeline window
// (LEAD chunks plus back-pressure slack).  When a wave owns several stripes (more
// than NW stripes) its ring is reused by its next stripe only after the consumer of
// the previous one has finished; that wait closes a chain of back-pressure waits
// through the other NW - 1 rings, which cannot stall as long as
// (NW - 1) * R > L2 + 64 + 4*STEP_QUANTUM.  A multiple of STEP_QUANTUM, hence of
// every chunk length.
__host__ inline int ring_len(int max_L1, int max_L2, int min_len) {
    const int ns = (max_L1 + 63) / 64;
    int r = min_len;
    if (ns > NW) {
        const int need = (max_L2 + 64 + 4 * STEP_QUANTUM + NW - 2) / (NW - 1) + 1;
        r = r > need ? r : need;
    }
    return (r + STEP_QUANTUM - 1) / STEP_QUANTUM * STEP_QUANTUM;
}

// Steps stored per stripe and plane in a skewed table: APAD leading steps t < 0,
// which the forward sweep fills with the column-0 boundary value (reverse sweeps
// read the cells left of column 0 from them without guards), then whole chunks.
__host__ __device__ inline int stored_steps(int L2max) {
    return APAD + ((L2max + 63 + STEP_QUANTUM - 1) / STEP_QUANTUM) * STEP_QUANTUM;
}

__host__ inline size_t status_bytes(int B) { return ((size_t)B * sizeof(int) + 255) / 256 * 256; }
__host__ inline size_t round256(size_t n) { return (n + 255) / 256 * 256; }

// Floats of `planes` skewed tables plus the last rows of every stripe per plane
// (B * stripes * planes * stored_steps * (64 + 1)).  elem_steps > 0: each element's
// table holds only elem_steps steps of 64 (a banded table); the last rows stay whole.
__host__ inline size_t table_floats(int B, int max_L1, int max_L2, int planes = 1,
                                    size_t elem_steps = 0) {
    const size_t ns = ((size_t)max_L1 + 63) / 64;
    const size_t rows = ns * (size_t)stored_steps(max_L2);
    return (size_t)B * planes * ((elem_steps ? elem_steps : rows) * 64 + rows);
}

// Workspace prefix of every entry point: per-element status words, the trash line,
// then the primal table(s) with their last rows.
struct Layout {
    int* status;
    float* trash;
    float* alpha_sk;   // [B][stripe][plane][step][64] (banded: [B][elem_steps][64])
    float* brow;       // [B][stripe][plane][step]
    size_t elem_steps; // table steps of 64 per element and plane
    // split elements (present when layout() is asked for them; up to one part per
    // stripe): progress words of the forward and reverse boundaries [B][stripe],
    // reverse-sweep boundary flows [B][stripe][step], per-part partial results
    uint64_t* fflag;
    uint64_t* bflag;
    float2* flows;     // (linear SW: float2 per step; affine: a float4 and a float
                       // plane of flow_slots each)
    size_t flow_slots; // B * stripes * stored steps
    float2* fpart;     // [B][stripe] (max, scaled sum) of the partition
    double* bpart;     // [B][stripe][4] parameter-gradient sums
    size_t bytes;      // bytes of this prefix
};

__host__ inline Layout layout(void* workspace, int B, int max_L1, int max_L2, int planes = 1,
                              bool split = false, int flow_bytes = 8, size_t elem_steps = 0) {
    Layout l;
    l.status = (int*)workspace;
    l.trash = (float*)((char*)workspace + status_bytes(B));
    l.alpha_sk = (float*)((char*)l.trash + TRASH_BYTES);
    const size_t ns = ((size_t)max_L1 + 63) / 64;
    l.elem_steps = elem_steps ? elem_steps : ns * (size_t)stored_steps(max_L2);
    l.brow = l.alpha_sk + (size_t)B * planes * l.elem_steps * 64;
    l.bytes = status_bytes(B) + TRASH_BYTES +
              table_floats(B, max_L1, max_L2, planes, elem_steps) * sizeof(float);
    l.fflag = l.bflag = nullptr;
    l.flows = l.fpart = nullptr;
    l.flow_slots = 0;
    l.bpart = nullptr;
    if (split) {
        char* p = (char*)workspace + round256(l.bytes);
        const size_t parts = (size_t)B * (ns > 0 ? ns : 1);
        l.fflag = (uint64_t*)p;
        p += round256(parts * sizeof(uint64_t));
        l.bflag = (uint64_t*)p;
        p += round256(parts * sizeof(uint64_t));
        l.flows = (float2*)p;
        l.flow_slots = parts * (size_t)stored_steps(max_L2);
        p += round256(l.flow_slots * (size_t)flow_bytes);
        l.fpart = (float2*)p;
        p += round256(parts * sizeof(float2));
        l.bpart = (double*)p;
        p += round256(parts * 4 * sizeof(double));
        l.bytes = (size_t)(p - (char*)workspace);
    }
    return l;
}

// Parts per element (G) and stripes per part (SPW) of a launch: G > 1 only when the
// layout has the split areas.  D2P_AMD_SPLIT=<n> in the environment forces n parts
// (at most one per stripe); unset or 0 chooses automatically.  max_spw > 0: the
// rings of an unsplit element do not fit in LDS, so no part may hold more than
// max_spw stripes (a part of at most NW stripes needs only the minimum ring).
struct Split {
    int G, SPW;
};
Split choose_split(int B, int max_L1, const Layout& ws, int max_spw = 0);

// Before a split forward sweep: status words and progress words to zero.
int launch_split_reset(const Layout& ws, int B, int G, hipStream_t st);
// Before every other split sweep: the n progress words it uses to zero (words the
// forward did not reset may hold anything, e.g. when this sweep has more parts).
int launch_flag_reset(uint64_t* flags, int n, hipStream_t st);
// After it: partition[b] from the parts' (max, scaled sum) in ws.fpart and the cell
// (0, 0), whose value is 0.
int launch_partition_merge(const Layout& ws, float* partition, int B, int G, float T,
                           hipStream_t st);
// The same, and sdot[b] = the value's tangent from the parts' tangent sums wpart[b][part]
// at their (max, scaled sum) scale (the cell (0, 0) adds a tangent of 0), weighted as
// 2^((alpha - S) c) with the fp32 partition S.
int launch_partition_dot_merge(const Layout& ws, const float* wpart, float* partition,
                               float* sdot, int B, int G, float T, hipStream_t st);
// out[b] = sum of the G parts' partial results spart[b][part].
int launch_sum_parts(const float* spart, float* out, int B, int G, hipStream_t st);

// The last launch of every entry point: each output of an element whose status word
// is set (one of its pipeline waits gave up, so its results rest on data that had
// not arrived) becomes NaN.  mats: up to two [B][per_elem] matrices, vecs: up to
// four [B] vectors; null pointers are skipped.  An element that is clean costs one
// load of its status word.
int launch_poison(const int* status, int B, long long per_elem, float* mat0, float* mat1,
                  float* vec0, float* vec1, float* vec2, float* vec3, hipStream_t st);

// Issue priority of a wave by its stripe's place in the pipeline: every stripe
// waits on the one before it, so the upstream stripes set the pace and are served
// first; downstream stripes fill the issue slots they leave.  `pos` = pipeline
// position of the stripe among those in flight (0 = most upstream).
__device__ __forceinline__ void set_pipeline_priority(int pos) {
    if (pos < 2) __builtin_amdgcn_s_setprio(3);
    else if (pos < 4) __builtin_amdgcn_s_setprio(2);
    else if (pos < 6) __builtin_amdgcn_s_setprio(1);
    else __builtin_amdgcn_s_setprio(0);
}

// ---------------------------------------------------------------- split elements

// An element's stripes may be divided among G workgroups ("parts"); part p owns the
// stripes [p*SPW, (p+1)*SPW).  Inside a part the stripes form the LDS pipeline below;
// between parts the boundary row (forward) or the boundary flows (reverse sweeps) go
// through global memory with device-coherent (sc0 sc1) accesses, and a per-part
// progress word ((epoch << 32) | chunks done) orders producer and consumer.  The
// epoch is new for every launch, so stale words of earlier launches never match.
// Workgroups are numbered so that the parts of one element share blockIdx % 8 (the
// XCD on MI355X: their boundary traffic stays in one L2 in practice; correctness
// does not depend on it) and every producer part has a lower index than its
// consumer, so it is dispatched first.
constexpr int XCDS = 8;

__host__ __device__ inline int split_grid(int B, int G) {
    return XCDS * ((B + XCDS - 1) / XCDS) * G;
}

// (element, part in dispatch order) of a workgroup; element >= B: idle workgroup.
__device__ __forceinline__ void split_decode(int bid, int G, int& b, int& part) {
    const int x = bid % XCDS, j = bid / XCDS;
    b = x + XCDS * (j / G);
    part = j % G;
}

// device-coherent global accesses (bypass the non-coherent caches)
__device__ __forceinline__ void store_sys(float* p, float v) {
    __asm__ volatile("global_store_dword %0, %1, off sc0 sc1" ::"v"(p), "v"(v) : "memory");
}
__device__ __forceinline__ void store_sys2(float2* p, float2 v) {
    __asm__ volatile("global_store_dwordx2 %0, %1, off sc0 sc1" ::"v"(p), "v"(v) : "memory");
}
__device__ __forceinline__ void store_flag(uint64_t* p, uint64_t v) {
    __asm__ volatile("global_store_dwordx2 %0, %1, off sc0 sc1" ::"v"(p), "v"(v) : "memory");
}
__device__ __forceinline__ uint64_t load_flag(const uint64_t* p) {
    uint64_t v;
    __asm__ volatile("global_load_dwordx2 %0, %1, off sc0 sc1\n\ts_waitcnt vmcnt(0)"
                     : "=v"(v) : "v"(p) : "memory");
    return v;
}
__device__ __forceinline__ int load_status(const int* p) {
    int v;
    __asm__ volatile("global_load_dword %0, %1, off sc0 sc1\n\ts_waitcnt vmcnt(0)"
                     : "=v"(v) : "v"(p) : "memory");
    return v;
}

// 16 bytes per lane, device-coherent
__device__ __forceinline__ void store_sys4(float4* p, float4 v) {
    typedef float f4 __attribute__((ext_vector_type(4)));
    const f4 w = {v.x, v.y, v.z, v.w};
    __asm__ volatile("global_store_dwordx4 %0, %1, off sc0 sc1" ::"v"(p), "v"(w) : "memory");
}

// Polls a pipeline wait makes before it gives up (this translation unit's copy, per
// device).  d2p_set_spin_limit lowers it from the host so that tests can drive every
// wait down its give-up path; kernels read it only once a wait is not satisfied at
// once, so the hot path never loads it.  It lives in constant memory: a kernel reads
// it with a scalar load, whose wait leaves the wave's vector-memory operations in
// flight (a vector load would be followed by a wait for all of them, draining the
// loads issued ahead and the stores just issued at every wait that is not satisfied
// at once).
static __constant__ int g_spin_limit = SPIN_LIMIT;

// Host side: every translation unit that includes this header registers a setter for
// its own copy of g_spin_limit (d2p_set_spin_limit calls them all).
void register_spin_setter(int (*setter)(int));
static int set_spin_limit_here(int spins) {
    return hipMemcpyToSymbol(HIP_SYMBOL(g_spin_limit), &spins, sizeof(int)) == hipSuccess ? 0 : -1;
}
static struct SpinSetterRegistration {
    SpinSetterRegistration() { register_spin_setter(&set_spin_limit_here); }
} g_spin_setter_registration;

// A progress word: the launch's epoch in the high half, the chunks done in the low.
__device__ __forceinline__ uint64_t progress_word(uint32_t epoch, int chunks) {
    return ((uint64_t)epoch << 32) | (uint32_t)chunks;
}

// Chunks a progress word reports for this epoch (-1: an earlier launch's word).
__device__ __forceinline__ int flag_chunks(uint64_t v, uint32_t epoch) {
    const uint32_t hi = __builtin_amdgcn_readfirstlane((uint32_t)(v >> 32));
    const uint32_t lo = __builtin_amdgcn_readfirstlane((uint32_t)v);
    return hi == epoch ? (int)lo : -1;
}

// A progress word prefetched one chunk ahead lands in the wave's 64-dword LDS slot
// (lane l loads dword min(l, 1) of the word), never in a VGPR: the compiler takes a
// VGPR written by an asynchronous load as defined when the load issues, and could
// copy it before the data arrives.  Read the slot with flag_chunks_lds after a
// vmcnt wait that covers the load, and before the next load into it.
__device__ __forceinline__ void flag_load_lds(const uint64_t* flag, uint32_t slot_lds, int lane);
__device__ __forceinline__ int flag_chunks_lds(const float* slot, uint32_t epoch) {
    const uint32_t lo = __float_as_uint(slot[0]), hi = __float_as_uint(slot[1]);
    return flag_chunks(((uint64_t)hi << 32) | lo, epoch);
}

// Waits until the part's progress word reports `need` chunks of this epoch; returns
// the chunks seen.  Bounded by a count of polls (a quarter of the spin limit; each
// poll is two device-coherent loads and a sleep, about 1 us), not by wall time, so a
// workgroup that is descheduled while it waits does not run its bound down.  On
// timeout, or when another wave of the element has already timed out, the element's
// status gets bit 0 and the wait gives up.
__device__ __forceinline__ int wait_part(const uint64_t* flag, uint32_t epoch, int need,
                                         int* status_b) {
    int got = flag_chunks(load_flag(flag), epoch);
    if (got >= need) return got;
    const int limit = max(__builtin_amdgcn_readfirstlane(g_spin_limit) >> 2, 1);
    for (int polls = 1;; ++polls) {
        if (__builtin_amdgcn_readfirstlane(load_status(status_b)) != 0) return need;
        if (polls >= limit) {
            atomicOr(status_b, 1);
            return need;
        }
        __builtin_amdgcn_s_sleep(8);
        got = flag_chunks(load_flag(flag), epoch);
        if (got >= need) return got;
    }
}

// ---------------------------------------------------------------- progress flags

// Progress flags live in LDS.  The writer completes its LDS writes (ring data)
// before the flag write; a reader that sees the flag issues its data reads after the
// flag read.  LDS executes each wave's operations in order, so relaxed atomics plus
// an LDS-only wait suffice (a C++ release/acquire would also drain every HBM load
// and store in flight).
__device__ __forceinline__ void publish(int* prog, int wave, int value) {
    wave_lds_sync();
    __hip_atomic_store(prog + wave, value, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
}

__device__ __forceinline__ int prog_load(int* prog, int w) {
    return __builtin_amdgcn_readfirstlane(
        __hip_atomic_load(prog + w, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP));
}

// Waits until prog[w] >= need; bounded by g_spin_limit polls, after which the
// element's status gets bit 0 and the wave goes on.  The loaded value is made
// wave-uniform.
__device__ __forceinline__ void wait_for(int* prog, int w, int need, int* status_b) {
    if (prog_load(prog, w) < need) {
        const int limit = __builtin_amdgcn_readfirstlane(g_spin_limit);
        int spins = 0;
        do {
            __builtin_amdgcn_s_sleep(2);
            if (++spins >= limit) {
                atomicOr(status_b, 1);
                break;
            }
        } while (prog_load(prog, w) < need);
    }
    wave_lds_sync();
}

// The chunk-level waits of sweep order q (q = stripe for forward sweeps, the
// reversed stripe index for reverse sweeps) before its chunk k: the producer q-1
// must be LEAD chunks ahead, and the consumer q+1 must have consumed the ring slots
// this chunk overwrites.  Before its first chunk (k_first: a stripe that sweeps only
// a window of its steps starts there), a stripe that reuses its wave's ring (q >= NW)
// also waits until the consumer of the ring's previous stripe (q - NW + 1) has
// finished.
template <int P>
__device__ __forceinline__ void chunk_waits(int* prog, int q, int NS, int k, int nch, int R,
                                            int* status_b, int k_first = 0) {
    if (k == k_first && q >= NW)
        wait_for(prog, (q + 1) % NW, (q - NW + 1) * PROG_STRIDE + nch, status_b);
    if (q > 0) wait_for(prog, (q - 1) % NW, (q - 1) * PROG_STRIDE + min(k + lead(P), nch), status_b);
    if (q + 1 < NS) {
        const int need = k - 2 - R / P;   // slots of steps < kP+P-R must be consumed
        if (need > 0) wait_for(prog, (q + 1) % NW, (q + 1) * PROG_STRIDE + need, status_b);
    }
}

// Progress words read one chunk ahead.  A sweep issues these LDS reads right after a
// chunk's steps, so that their latency overlaps the rest of that chunk's work; at the
// next chunk's start, a wait whose condition the value read already meets costs a
// compare.  The values may be stale, but progress only grows, so a condition they meet
// holds; one they do not meet falls back to wait_for.  The reads stay in VGPRs until
// the compare (a readfirstlane right after each read would wait for it at once).
struct ProgAhead {
    int prod, cons, help;   // the producer's and consumer's words, the helper's chunks
};
__device__ __forceinline__ int prog_peek(int* prog, int w) {
    return __hip_atomic_load(prog + w, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
}
__device__ __forceinline__ void prog_ahead(ProgAhead& a, int* prog, int* hprog, int q, int NS,
                                           int h) {
    a.prod = q > 0 ? prog_peek(prog, (q - 1) % NW) : 0;
    a.cons = q + 1 < NS ? prog_peek(prog, (q + 1) % NW) : 0;
    a.help = hprog != nullptr ? prog_peek(hprog, h) : 0;
}
__device__ __forceinline__ void prog_ahead_reset(ProgAhead& a) { a.prod = a.cons = a.help = -1; }
// wait_for(prog, w, need, ...) unless the value read ahead already shows need
__device__ __forceinline__ void wait_for_ahead(int seen, int* prog, int w, int need,
                                               int* status_b) {
    if (__builtin_amdgcn_readfirstlane(seen) < need) wait_for(prog, w, need, status_b);
}
// chunk_waits with the producer's and consumer's words read ahead
template <int P>
__device__ __forceinline__ void chunk_waits_ahead(const ProgAhead& a, int* prog, int q, int NS,
                                                  int k, int nch, int R, int* status_b) {
    if (k == 0 && q >= NW)
        wait_for(prog, (q + 1) % NW, (q - NW + 1) * PROG_STRIDE + nch, status_b);
    if (q > 0)
        wait_for_ahead(a.prod, prog, (q - 1) % NW,
                       (q - 1) * PROG_STRIDE + min(k + lead(P), nch), status_b);
    if (q + 1 < NS) {
        const int need = k - 2 - R / P;   // slots of steps < kP+P-R must be consumed
        if (need > 0)
            wait_for_ahead(a.cons, prog, (q + 1) % NW, (q + 1) * PROG_STRIDE + need, status_b);
    }
}

__device__ __forceinline__ int ring_index(int slot, int R) {
    slot %= R;
    return slot < 0 ? slot + R : slot;
}

// One ring of R elements of type E per wave ([NW][R]): the ring sweep order q
// writes, and the ring it reads (written by q - 1).
template <class E>
__device__ __forceinline__ E* ring_of(E* rings, int q, int R) {
    return rings + (q % NW) * R;
}
template <class E>
__device__ __forceinline__ E* ring_from(E* rings, int q, int R) {
    return rings + ((q + NW - 1) % NW) * R;
}

// ------------------------------------------------------------ direct-to-LDS loads

// One dword per lane straight from HBM into LDS (global_load_lds_dword): lane l's
// value lands at LDS byte address lds + 4*l; the LDS address travels in M0.  Each
// call then advances `lds` by LDS_STEP and `voff` by `vstep` bytes.  Inline assembly,
// so that (a) the compiler does not make every later LDS access wait for the load
// (completion is waited for explicitly with wait_vmcnt), and (b) the running
// addresses stay in two registers instead of being hoisted out of the loop as one
// precomputed address per instruction.
// M0 is a reserved register the compiler may use itself (LDS-DMA builtins, indexed
// register moves); these kernels use neither, so clobbering it here is safe, and the
// compiler's reminder about reserved clobbers is silenced.
#pragma clang diagnostic push
#pragma clang diagnostic ignored "-Winline-asm"
template <int LDS_STEP>
__device__ __forceinline__ void lds_dma_dword(const float* sbase, uint32_t& voff, uint32_t& lds,
                                              uint32_t vstep) {
    __asm__ volatile(
        "s_mov_b32 m0, %1\n\t"
        "s_nop 0\n\t"
        "global_load_lds_dword %0, %2\n\t"
        "s_add_u32 %1, %1, %4\n\t"
        "v_add_u32 %0, %3, %0"
        : "+v"(voff), "+s"(lds)
        : "s"(sbase), "s"(vstep), "n"(LDS_STEP)
        : "memory", "m0", "scc");
}
// The same with device-coherent (sc0 sc1) reads, for data another workgroup wrote
// during this launch.
template <int LDS_STEP>
__device__ __forceinline__ void lds_dma_dword_sys(const float* sbase, uint32_t& voff,
                                                  uint32_t& lds, uint32_t vstep) {
    __asm__ volatile(
        "s_mov_b32 m0, %1\n\t"
        "s_nop 0\n\t"
        "global_load_lds_dword %0, %2 sc0 sc1\n\t"
        "s_add_u32 %1, %1, %4\n\t"
        "v_add_u32 %0, %3, %0"
        : "+v"(voff), "+s"(lds)
        : "s"(sbase), "s"(vstep), "n"(LDS_STEP)
        : "memory", "m0", "scc");
}

// The same with 16 bytes per lane: lane l's four dwords land at LDS M0 + 16*l.
template <int LDS_STEP>
__device__ __forceinline__ void lds_dma_dwordx4(const float* sbase, uint32_t& voff, uint32_t& lds,
                                                uint32_t vstep) {
    __asm__ volatile(
        "s_mov_b32 m0, %1\n\t"
        "s_nop 0\n\t"
        "global_load_lds_dwordx4 %0, %2\n\t"
        "s_add_u32 %1, %1, %4\n\t"
        "v_add_u32 %0, %3, %0"
        : "+v"(voff), "+s"(lds)
        : "s"(sbase), "s"(vstep), "n"(LDS_STEP)
        : "memory", "m0", "scc");
}
// The same, marked non-temporal: for data read exactly once (the skewed tables), so
// that it does not push reused lines (the score rows of the next chunk) out of L2.
template <int LDS_STEP>
__device__ __forceinline__ void lds_dma_dwordx4_nt(const float* sbase, uint32_t& voff,
                                                   uint32_t& lds, uint32_t vstep) {
    __asm__ volatile(
        "s_mov_b32 m0, %1\n\t"
        "s_nop 0\n\t"
        "global_load_lds_dwordx4 %0, %2 nt\n\t"
        "s_add_u32 %1, %1, %4\n\t"
        "v_add_u32 %0, %3, %0"
        : "+v"(voff), "+s"(lds)
        : "s"(sbase), "s"(vstep), "n"(LDS_STEP)
        : "memory", "m0", "scc");
}
#pragma clang diagnostic pop

__device__ __forceinline__ void flag_load_lds(const uint64_t* flag, uint32_t slot_lds, int lane) {
    uint32_t voff = lane > 0 ? 4u : 0u;
    lds_dma_dword_sys<0>(reinterpret_cast<const float*>(flag), voff, slot_lds, 0u);
}

// Waits until at most N vector-memory operations of this wave are outstanding
// (gfx9 counts loads, stores and LDS DMA on one in-order counter).
template <int N>
__device__ __forceinline__ void wait_vmcnt() {
    static_assert(N >= 0 && N < 64, "vmcnt range");
    __asm__ volatile("s_waitcnt vmcnt(%0)" ::"n"(N) : "memory");
}

__device__ __forceinline__ uint32_t lds_address(const void* p) {
    return (uint32_t)(uintptr_t)p;   // low half of a flat LDS address = LDS offset
}

// Accesses base + byte offset with a wave-uniform base and a 32-bit per-lane offset,
// the form the scalar-base global instructions take (no 64-bit address per lane).
__device__ __forceinline__ float lane_load(const float* base, unsigned off_bytes) {
    return *reinterpret_cast<const float*>(reinterpret_cast<const char*>(base) + off_bytes);
}
__device__ __forceinline__ void lane_store(float* base, unsigned off_bytes, float v) {
    *reinterpret_cast<float*>(reinterpret_cast<char*>(base) + off_bytes) = v;
}

// ------------------------------------------------------------ chunk tiles

// A chunk covers P steps of a stripe's 64 rows; cell (row r, step u) is column
// t_first + DIR*u - r of DP row i0 + r (DIR = +1 forward, -1 reverse sweep).
//
// Tiles of per-cell matrices are staged with P direct-to-LDS loads: instruction i,
// lane P*j+u carries row r = i+P*j, step u, and lands at float 65*i + P*j + u of the
// tile.  Row r, step u is therefore at 65*(r%P) + P*(r/P) + u, whose bank (mod 64)
// is r+u: the per-step column read of the 64 lanes is conflict-free.  Output tiles
// use the same layout, and instruction i of the write-out stores tile floats
// 65*i .. 65*i+63.
template <int P>
struct ChunkTile {
    static_assert(64 % P == 0, "chunk length must divide 64");
    static constexpr int FLOATS = 65 * P;
    __device__ static int read_base(int lane) { return 65 * (lane % P) + P * (lane / P); }
};

// True when every cell of the chunk lies inside the (max_L1 x max_L2) matrix.  Then
// cell addresses of instruction i are the lane's address of instruction 0 plus
// i*(L2max-1): one wave-uniform increment, no per-lane clamping.
template <int P, int DIR>
__device__ __forceinline__ bool chunk_inside(int i0, int L1max, int L2max, int t_first) {
    const int lo = DIR > 0 ? t_first - 63 : t_first - (P - 1) - 63;
    const int hi = DIR > 0 ? t_first + P - 1 : t_first;
    return lo >= 0 && hi < L2max && i0 + 63 < L1max;
}

// Offset (floats) of the lane's cell of instruction 0 from the stripe's first row.
// The tile helpers address a matrix from the wave-uniform row pointer of the stripe
// (stripe_row), so a lane offset spans at most 64 rows whatever the element's size.
template <int P, int DIR>
__device__ __forceinline__ int chunk_offset0(int L2max, int lane, int t_first) {
    const int u = lane % P, pj = lane - u;
    return pj * L2max + t_first + DIR * u - pj;
}

template <class T>
__device__ __forceinline__ T* stripe_row(T* mbase, int i0, int L2max) {
    return mbase + (size_t)i0 * L2max;
}

// Issues the P loads of one chunk of a row-major [L1max][L2max] matrix into a tile.
// Cells outside the matrix read a clamped in-matrix address; the sweeps mask every
// cell outside the element's lengths.
template <int P, int DIR>
__device__ __forceinline__ void dma_tile(uint32_t tile_lds, const float* mbase, int i0, int L1max,
                                         int L2max, int lane, int t_first) {
    const float* sbase = stripe_row(mbase, i0, L2max);
    if (chunk_inside<P, DIR>(i0, L1max, L2max, t_first)) {
        uint32_t voff = (uint32_t)chunk_offset0<P, DIR>(L2max, lane, t_first) * 4u;
        const uint32_t vstep = (uint32_t)(L2max - 1) * 4u;
#pragma unroll
        for (int i = 0; i < P; ++i) lds_dma_dword<260>(sbase, voff, tile_lds, vstep);
    } else {
        const int u = lane % P, pj = lane - u;
        // row/column of instruction 0; instruction i moves one row down, one column left
        int row = i0 + pj, col = t_first + DIR * u - pj;
#pragma unroll
        for (int i = 0; i < P; ++i) {
            uint32_t voff = (uint32_t)((min(row, L1max - 1) - i0) * L2max +
                                       min(max(col, 0), L2max - 1)) * 4u;
            lds_dma_dword<260>(sbase, voff, tile_lds, 0u);
            ++row;
            --col;
        }
    }
}


// Writes a chunk's output tile back to a row-major [L1max][L2max] matrix: exactly P
// stores.  Inside chunks write every cell (cells outside the element's lengths must
// hold 0 in the tile); boundary chunks send the cells outside the element's lengths
// to the trash line.
template <int P, int DIR>
__device__ __forceinline__ void write_tile(const float* tile, float* obase, float* trash, int i0,
                                           int L1, int L2, int L1max, int L2max, int lane,
                                           int t_first) {
    if (chunk_inside<P, DIR>(i0, L1max, L2max, t_first)) {
        float* sbase = stripe_row(obase, i0, L2max);
        uint32_t off4 = (uint32_t)chunk_offset0<P, DIR>(L2max, lane, t_first) * 4u;
        const uint32_t step4 = (uint32_t)(L2max - 1) * 4u;
        // all LDS reads first (one wait), then the stores: the empty asm that keeps
        // one running offset would otherwise order each read behind the last store
        float v[P];
#pragma unroll
        for (int i = 0; i < P; ++i) v[i] = tile[65 * i + lane];
#pragma unroll
        for (int i = 0; i < P; ++i) {
            lane_store(sbase, off4, v[i]);
            off4 += step4;
            __asm__ volatile("" : "+v"(off4));   // keep one running offset
        }
    } else {
        const int u = lane % P, pj = lane - u;
        int row = i0 + pj, col = t_first + DIR * u - pj;
#pragma unroll
        for (int i = 0; i < P; ++i) {
            const bool in = row < L1 && col >= 0 && col < L2;
            float* dst = in ? obase + (size_t)row * L2max + col : trash + lane;
            *dst = tile[65 * i + lane];
            ++row;
            --col;
        }
    }
}

// ------------------------------------------------------------ quad tiles

// A chunk of P steps (P = 8 or 16) of a stripe's 64 rows staged with 16-byte
// direct-to-LDS loads: row r occupies P consecutive floats; its quad q (steps
// 4q .. 4q+3) sits at slot q ^ swz(r), the four values in memory-column order
// (ascending steps for DIR = +1, descending for DIR = -1).  swz spreads the 16
// lanes of one LDS pass over all 64 banks, so the per-lane 16-byte row reads are
// conflict-free.  An inside chunk takes P/4 loads (instruction i: lane l carries
// the 16 bytes at tile float 256*i + 4*l); a boundary chunk takes P clamped dword
// loads into the same layout.  Output tiles use the same layout.
template <int P>
struct QuadTile {
    // swz has a period of 16 rows, which divides the 64/NQ rows one 16-byte
    // instruction covers: successive instructions see the same swizzle per lane (the
    // running-offset loads rely on it)
    static_assert(P == 8 || P == 16, "quad tiles hold 8 or 16 steps");
    static constexpr int FLOATS = 64 * P;
    static constexpr int NQ = P / 4;                // quads per row
    static constexpr int ROWS_X4 = 64 / NQ;         // rows per 16-byte instruction
    __device__ static int swz(int r) { return (int)(((unsigned)r / (16 / NQ)) & (NQ - 1)); }
    __device__ static int slot(int r, int q) { return P * r + 4 * (q ^ swz(r)); }
    // step of element e of the quad q
    template <int DIR>
    __device__ static constexpr int step(int q, int e) { return DIR > 0 ? 4 * q + e : 4 * q + 3 - e; }
};

// (row, column) of tile float f = 64*j + lane of the dword form, relative to i0.
template <int P, int DIR>
__device__ __forceinline__ void quad_cell(int f, int t_first, int& r, int& col) {
    using Q = QuadTile<P>;
    r = (int)((unsigned)f / P);   // f >= 0: unsigned division is a shift
    const int s = (int)((unsigned)f % P);
    const int q = (s >> 2) ^ Q::swz(r);
    col = t_first + DIR * Q::template step<DIR>(q, s & 3) - r;
}

// Byte offset from the stripe's first row (stripe_row) of the 16 bytes an inside
// chunk's instruction 0 moves for this lane (the lowest column of the lane's quad);
// instruction i adds i * ROWS_X4 * (L2max - 1) floats.
template <int P, int DIR>
__device__ __forceinline__ uint32_t quad_offset0(int L2max, int lane, int t_first) {
    using Q = QuadTile<P>;
    const int r = lane / Q::NQ;
    const int q = (lane % Q::NQ) ^ Q::swz(r);
    const int c_lo = DIR > 0 ? t_first + 4 * q - r : t_first - 4 * q - 3 - r;
    return (uint32_t)(r * L2max + c_lo) * 4u;
}

// Issues the loads of one chunk of a row-major [L1max][L2max] matrix into a quad tile.
template <int P, int DIR>
__device__ __forceinline__ void dma_quads(uint32_t tile_lds, const float* mbase, int i0,
                                          int L1max, int L2max, int lane, int t_first) {
    using Q = QuadTile<P>;
    const float* sbase = stripe_row(mbase, i0, L2max);
    if (chunk_inside<P, DIR>(i0, L1max, L2max, t_first)) {
        uint32_t voff = quad_offset0<P, DIR>(L2max, lane, t_first);
        const uint32_t vstep = (uint32_t)(Q::ROWS_X4 * (L2max - 1)) * 4u;
#pragma unroll
        for (int i = 0; i < Q::NQ; ++i) lds_dma_dwordx4<1024>(sbase, voff, tile_lds, vstep);
    } else {
#pragma unroll
        for (int j = 0; j < P; ++j) {
            int r, col;
            quad_cell<P, DIR>(64 * j + lane, t_first, r, col);
            uint32_t voff = (uint32_t)((min(i0 + r, L1max - 1) - i0) * L2max +
                                       min(max(col, 0), L2max - 1)) * 4u;
            lds_dma_dword<256>(sbase, voff, tile_lds, 0u);
        }
    }
}

// The lane's P values (row = lane), in step order.
template <int P, int DIR>
__device__ __forceinline__ void read_quads(const float* tile, int lane, float (&v)[P]) {
    using Q = QuadTile<P>;
#pragma unroll
    for (int q = 0; q < Q::NQ; ++q) {
        const float4 x = *reinterpret_cast<const float4*>(tile + Q::slot(lane, q));
        v[Q::template step<DIR>(q, 0)] = x.x;
        v[Q::template step<DIR>(q, 1)] = x.y;
        v[Q::template step<DIR>(q, 2)] = x.z;
        v[Q::template step<DIR>(q, 3)] = x.w;
    }
}

// Stores the lane's values of quad q (steps 4q .. 4q+3) into its row of the tile.
template <int P, int DIR>
__device__ __forceinline__ void put_quad(float* tile, int lane, int q, const float* v) {
    using Q = QuadTile<P>;
    float4 x;
    x.x = v[Q::template step<DIR>(q, 0)];
    x.y = v[Q::template step<DIR>(q, 1)];
    x.z = v[Q::template step<DIR>(q, 2)];
    x.w = v[Q::template step<DIR>(q, 3)];
    *reinterpret_cast<float4*>(tile + Q::slot(lane, q)) = x;
}

// Writes a quad tile back to a row-major [L1max][L2max] matrix: P/4 16-byte stores
// for an inside chunk (cells outside the element's lengths must hold 0), P dword
// stores for a boundary chunk (cells outside the lengths go to the trash line).
template <int P, int DIR>
__device__ __forceinline__ void write_quads(const float* tile, float* obase, float* trash, int i0,
                                            int L1, int L2, int L1max, int L2max, int lane,
                                            int t_first) {
    using Q = QuadTile<P>;
    if (chunk_inside<P, DIR>(i0, L1max, L2max, t_first)) {
        char* sbase = reinterpret_cast<char*>(stripe_row(obase, i0, L2max));
        uint32_t off = quad_offset0<P, DIR>(L2max, lane, t_first);
        const uint32_t step = (uint32_t)(Q::ROWS_X4 * (L2max - 1)) * 4u;
#pragma unroll
        for (int i = 0; i < Q::NQ; ++i) {
            const float4 v = *reinterpret_cast<const float4*>(tile + 256 * i + 4 * lane);
            *reinterpret_cast<float4*>(sbase + off) = v;
            off += step;
            __asm__ volatile("" : "+v"(off));   // keep one running offset
        }
    } else {
        // one value at a time: boundary chunks are few, and the kernels that call this
        // run near their register budget
#pragma unroll
        for (int j = 0; j < P; ++j) {
            int r, col;
            quad_cell<P, DIR>(64 * j + lane, t_first, r, col);
            const int row = i0 + r;
            const bool in = row < L1 && col >= 0 && col < L2;
            // (the offset stays below L1max * L2max < 2^31)
            float* dst = in ? obase + (uint32_t)(row * L2max + col) : trash + lane;
            *dst = tile[64 * j + lane];
        }
    }
}

// Aligned write-out of a reverse sweep's output tiles of P = 8 or 16 steps (quad tiles,
// QUAD, or dword chunk tiles), for matrices whose rows start P-float aligned (L2max %
// P == 0; a P-float segment is then two or one whole 32-byte sectors).  Chunk t_hi of
// row r covers columns c - (P - 1) .. c (c = t_hi - r); the row's aligned segment
// [a, a + P - 1], a = c & ~(P - 1), takes its columns <= c from this chunk's tile and the
// others from the previous chunk's, which the caller keeps in `carry` from the previous
// call (zeros before a stripe's first chunk: those columns lie past the element).  Each
// row therefore gets exactly one whole segment per chunk, and a stripe's chunks cover
// every segment of its rows.  Lane l moves quarter l % (P/4) of the segments of rows
// (64/(P/4)) i + l / (P/4), one 16-byte store each (P/4 stores, as write_quads); a
// segment outside the matrix goes to the trash line.  Cells outside the element must
// hold 0 in the tiles.
typedef float f32x4 __attribute__((ext_vector_type(4)));
template <int P>
struct AlignedCarry {
    f32x4 v[P / 4];
    __device__ void clear() {
#pragma unroll
        for (int i = 0; i < P / 4; ++i) v[i] = (f32x4){0.0f, 0.0f, 0.0f, 0.0f};
    }
};
template <int P, bool QUAD>
__device__ __forceinline__ void write_aligned(const float* tile, float* obase, float* trash,
                                              AlignedCarry<P>& cy, int i0, int L1max, int L2max,
                                              int lane, int t_hi) {
    static_assert(P == 8 || P == 16, "aligned write-out of 8- or 16-step tiles");
    constexpr int NQ = P / 4, RPI = 64 / NQ;   // slots per lane, rows per instruction
#pragma unroll
    for (int i = 0; i < NQ; ++i) {
        const int r = RPI * i + lane / NQ, p = lane % NQ;
        const int c = t_hi - r;
        const int a = c & ~(P - 1);
        const int u0 = (c & (P - 1)) - 4 * p;   // element e is step u0 - e of this chunk
        f32x4 out;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            const int u1 = u0 - e;               // < 0: the previous chunk's step u1 + P
            const int u = u1 & (P - 1);
            const float rd = QUAD ? tile[QuadTile<P>::slot(r, u >> 2) + 3 - (u & 3)]
                                  : tile[65 * (r % P) + P * (r / P) + u];
            out[e] = u1 >= 0 ? rd : cy.v[i][e];
            cy.v[i][e] = rd;                     // the next segment's share of this chunk
        }
        const bool in = a >= 0 && a + P - 1 < L2max && i0 + r < L1max;
        float* dst = in ? obase + (size_t)(i0 + r) * L2max + a + 4 * p : trash + 4 * (lane & 15);
        *reinterpret_cast<f32x4*>(dst) = out;
    }
}

// Register staging of a chunk's quad tile, for helper waves that load further ahead
// than their LDS buffers allow: stage_quads issues the loads dma_quads would issue,
// into the lane's registers (P/4 16-byte loads inside, P dword loads at a boundary),
// and put_staged_quads writes them where dma_quads would have put them.  The compiler
// tracks these loads itself and waits for them before the LDS writes.  The quads are
// held as vectors: as scalars, the compiler would split each 16-byte load into four
// and merge them with the boundary form's loads.
template <int P>
struct StagedQuads {
    f32x4 q[P / 4];
    bool inside;
};
template <int P, int DIR>
__device__ __forceinline__ void stage_quads(StagedQuads<P>& sq, const float* mbase, int i0,
                                            int L1max, int L2max, int lane, int t_first) {
    using Q = QuadTile<P>;
    const float* sbase = stripe_row(mbase, i0, L2max);
    sq.inside = chunk_inside<P, DIR>(i0, L1max, L2max, t_first);
    if (sq.inside) {
        const char* cbase = reinterpret_cast<const char*>(sbase);
        uint32_t off = quad_offset0<P, DIR>(L2max, lane, t_first);
        const uint32_t step = (uint32_t)(Q::ROWS_X4 * (L2max - 1)) * 4u;
#pragma unroll
        for (int i = 0; i < Q::NQ; ++i) {
            // (a 4-byte aligned address: 16-byte loads need no more on this part)
            sq.q[i] = *reinterpret_cast<const f32x4*>(cbase + off);
            off += step;
        }
    } else {
#pragma unroll
        for (int j = 0; j < P; ++j) {
            int r, col;
            quad_cell<P, DIR>(64 * j + lane, t_first, r, col);
            // (the offset stays below L1max * L2max < 2^31)
            sq.q[j / 4][j % 4] = sbase[(uint32_t)((min(i0 + r, L1max - 1) - i0) * L2max +
                                                  min(max(col, 0), L2max - 1))];
        }
    }
}
template <int P>
__device__ __forceinline__ void put_staged_quads(float* tile, const StagedQuads<P>& sq, int lane) {
    if (sq.inside) {
#pragma unroll
        for (int i = 0; i < P / 4; ++i) reinterpret_cast<f32x4*>(tile)[64 * i + lane] = sq.q[i];
    } else {
#pragma unroll
        for (int j = 0; j < P; ++j) tile[64 * j + lane] = sq.q[j / 4][j % 4];
    }
}

// Register staging of P consecutive steps of the lane's own row (row i0 + lane) of a
// row-major [L1max][L2max] matrix: step t_first + j is column t_first + j - lane.  A
// chunk inside the matrix takes P/4 16-byte loads per lane (4-byte aligned), one at a
// boundary P dword loads from clamped addresses (the sweeps mask those cells).
template <int P>
__device__ __forceinline__ void stage_row(f32x4 (&v)[P / 4], const float* mbase, int i0,
                                          int L1max, int L2max, int lane, int t_first) {
    const float* sbase = stripe_row(mbase, i0, L2max);
    if (i0 + 63 < L1max && t_first - 63 >= 0 && t_first + P - 1 < L2max) {
        const char* cbase = reinterpret_cast<const char*>(sbase);
        // (the offset spans at most 64 rows)
        const uint32_t off = (uint32_t)(lane * (L2max - 1) + t_first) * 4u;
#pragma unroll
        for (int i = 0; i < P / 4; ++i)
            v[i] = *reinterpret_cast<const f32x4*>(cbase + off + 16u * (uint32_t)i);
    } else {
        const int r = min(i0 + lane, L1max - 1) - i0;
#pragma unroll
        for (int j = 0; j < P; ++j) {
            const int col = min(max(t_first + j - lane, 0), L2max - 1);
            v[j / 4][j % 4] = sbase[(uint32_t)(r * L2max + col)];
        }
    }
}

// Register staging of dma_rows: the same P/4 non-temporal 16-byte loads per lane, and
// the LDS writes that put them where dma_rows would.
template <int P, int DIR>
__device__ __forceinline__ void stage_rows(f32x4 (&a)[P / 4], const float* plane_base, int t_first,
                                           int lane) {
    static_assert(P % 4 == 0, "rows come in fours");
    const int t_lo = DIR > 0 ? t_first : t_first - (P - 1);
    const f32x4* src = reinterpret_cast<const f32x4*>(plane_base + (size_t)(t_lo + APAD) * 64) + lane;
#pragma unroll
    for (int j = 0; j < P / 4; ++j) a[j] = __builtin_nontemporal_load(src + 64 * j);
}
template <int P>
__device__ __forceinline__ void put_staged_rows(float* rows, const f32x4 (&a)[P / 4], int lane) {
#pragma unroll
    for (int j = 0; j < P / 4; ++j) reinterpret_cast<f32x4*>(rows)[64 * j + lane] = a[j];
}

// Issues the loads of P consecutive steps of one plane of a skewed table (plane_base =
// the plane's step -APAD) into P LDS rows of 64, with 16-byte non-temporal loads
// (four 256-byte step rows per instruction, P/4 instructions).  LDS row j then holds
// step t_first + j for DIR = +1 and step t_first - (P - 1) + j for DIR = -1; read
// step t_first + DIR*j at row rows_row<P, DIR>(j).
template <int P, int DIR>
__device__ __forceinline__ void dma_rows(uint32_t rows_lds, const float* plane_base, int t_first,
                                         unsigned ul4) {
    static_assert(P % 4 == 0, "rows come in fours");
    const int t_lo = DIR > 0 ? t_first : t_first - (P - 1);
    uint32_t voff = (uint32_t)(t_lo + APAD) * 256u + 4u * ul4;
#pragma unroll
    for (int j = 0; j < P / 4; ++j) lds_dma_dwordx4_nt<1024>(plane_base, voff, rows_lds, 1024u);
}
template <int P, int DIR>
__device__ __host__ constexpr int rows_row(int j) { return DIR > 0 ? j : P - 1 - j; }

// Zeroes the cells of a row-major [L1max][L2max] output outside [0,L1) x [0,L2) in
// rows [r_begin, r_end) (default: all), with all threads of the workgroup.
__device__ __forceinline__ void zero_padding(float* obase, int L1, int L2, int L1max, int L2max,
                                             int nthreads, int r_begin = 0, int r_end = -1) {
    if (L1 >= L1max && L2 >= L2max) return;
    if (r_end < 0) r_end = L1max;
    for (int r = r_begin; r < r_end; ++r) {
        const int c0 = r < L1 ? L2 : 0;
        for (int c = c0 + (int)threadIdx.x; c < L2max; c += nthreads)
            obase[(size_t)r * L2max + c] = 0.0f;
    }
}

}  // namespace wf
}  // namespace d2p_amd
