// The whole decode step of one sequence (B = 1) as one persistent gfx950 kernel.
//
// Reference: engine/engine.py:805-839 (_forward_decode, one captured step) with
// the block of engine/engine.py:665-736 and the op semantics of
// engine/kernels/fused.py (add_norm :115-158, norm_rope :161-251, kv_to_cache
// :553-638, decode attention + split merge :641-846, swiglu :89-112) and
// argmax (engine/engine.py:833).
//
// At batch 1 a step streams 8 GB of weights through ~180 dependent ops.  With
// one kernel per op, every op boundary drains HBM: the next op's weight loads
// cannot start before its input exists.  Here one workgroup per CU lives for the
// whole step, and the weight stream never waits for an op boundary:
//
//  * waves 0..NLOAD-1 ("loaders") walk this workgroup's rows of every weight
//    matrix of the step in order -- qkv, o, gate/up, down of each layer, then
//    the LM head -- and copy them, 1 KB unit by unit, straight from HBM into a
//    96 KB LDS ring (global_load_lds), LDEPTH units in flight per wave.  Units
//    of the next matrix go out while the current one's output is still being
//    exchanged between workgroups; a slot is refilled once the unit in it has
//    been consumed.  The loaders never read what they load, so no wait of
//    theirs depends on the consumers' pace.
//  * waves NLOAD..NLOAD+NCOMP-1 ("compute") take rows in turn and read them
//    from the ring.  A row's dot product is summed per lane over its
//    512-element chunks in order and then across the wave: the arithmetic and
//    order of the GEMV kernel (q3_gemv), so every projection matches it bit for
//    bit.
//  * the last wave ("control") does everything else: it gathers each matrix's
//    input vector into LDS (RMSNorm'd where the op has a norm, with the GEMV
//    prologue's summation order), releases it to the compute waves through an
//    LDS counter, applies the epilogue to their row sums (residual add,
//    SwiGLU, argmax) and publishes this workgroup's outputs; per layer it also
//    runs one (KV head, key range) unit of attention -- q/k RMSNorm + RoPE and
//    the KV append fused in -- and one slice of the split merge.
//
// Exchange between workgroups: every published value travels as 32-bit words
// (16 payload bits | 16-bit flag << 16) stored and loaded device-coherently
// (sc1: past the XCD-private L2s).  A consumer re-reads until every word it
// needs carries the flag of the current (step, layer, op), so the data is its
// own ready signal -- one store and one load per dependency, no counter round
// trip, no L2 write-back or invalidate.  Flags only need to differ between
// consecutive writes of one buffer (each write waits, through the op chain,
// for every read of the previous one); the step epoch in state[0] keeps them
// distinct across steps and calls.
//
// Every wait is bounded in time.  On a timeout (a grid that is not fully
// resident, a device fault elsewhere) the workgroup records an error in
// state[1], writes token -1 and exits; nothing spins forever.
#include <utility>

#include "q3_attn_mfma.hpp"
#include "q3_common.hpp"
#include "q3_exchange.hpp"
#include "q3.h"

namespace {

using namespace q3x;

constexpr int PD = 128;               // head_dim
constexpr int PGROUP = 4;             // query heads per KV head
constexpr int CHUNK = 512;            // BF16 elements per streamed unit: 64 lanes x 16 bytes
constexpr int NWAVES = 8;
constexpr int PTHREADS = NWAVES * Q3_WAVE;
constexpr int NLOAD = 3;              // loader waves 0..2: weights HBM -> LDS ring
constexpr int NCOMP = 4;              // compute waves 3..6: ring x input -> row sums
constexpr int CTL_WAVE = NLOAD + NCOMP;  // wave 7: exchange, norms, epilogues, attention
static_assert(CTL_WAVE == NWAVES - 1, "wave roles");
#ifndef Q3_PERSIST_RU
#define Q3_PERSIST_RU 96
#endif
constexpr int RU = Q3_PERSIST_RU;     // ring units (1 KB each) in LDS
#ifndef Q3_PERSIST_LDEPTH
#define Q3_PERSIST_LDEPTH 8
#endif
constexpr int LDEPTH = Q3_PERSIST_LDEPTH;  // ring loads in flight per loader wave
constexpr int MAX_X = 10240;          // staged input elements (LDS)
constexpr int MAX_ROWS = 1024;        // row sums per workgroup per matrix
constexpr int MAX_OWN = 64;           // residual rows owned per workgroup
constexpr int PREC = 264;             // words per attention partial: acc[128], m, l as (hi, lo) pairs, padded
constexpr int MAX_SPLITS = 128;       // key ranges per KV head (two per merge lane)
constexpr int MAX_SLICE = 16;         // merged outputs per workgroup
constexpr int STAGE_CHUNKS = 10;      // 8-element chunks per lane gathered per round trip
constexpr int ATT_KEYS = 64;          // cached keys gathered into LDS per round trip: two 32-key tiles
constexpr int LDS_BYTES = 160 * 1024; // the whole CU's LDS: one workgroup per CU
constexpr uint64_t CTL_TIMEOUT = 100000000ull;     // wall-clock ticks (100 MHz): 1 s
constexpr uint64_t STREAM_TIMEOUT = 200000000ull;  // 2 s: longer than any single control wait

enum { OP_QKV = 0, OP_ATTN, OP_MERGE, OP_O, OP_GU, OP_DOWN, OP_COUNT = 8 };

// Optional step trace (wall clock, 100 MHz): TRACE_WGS workgroups (0, 1, G/2,
// G-1) record, per layer, TRACE_EV control-wave events; per streamed matrix,
// for compute wave 0, when it began waiting for the input and when it saw it,
// and for loader 0, when it issued the matrix's first unit.
constexpr int TRACE_WGS = 4;
constexpr int TRACE_EV = 16;
enum {
    T_QKV_IN = 0,   // qkv input gathered (residual ready)
    T_QKV_DONE,     // compute waves finished qkv
    T_ATT_IN,       // q/k/v of this head ready
    T_ATT_DONE,     // partial published
    T_MRG_IN,       // partials ready
    T_MRG_DONE,     // merged slice published
    T_O_IN,         // o input gathered
    T_O_DONE,
    T_GU_IN,
    T_GU_DONE,
    T_DN_IN,
    T_DN_DONE,
    T_START = 15,   // layer 0 only: control wave start
};
__host__ __device__ constexpr int trace_words(int L) {
    return TRACE_WGS * ((L + 1) * TRACE_EV + 3 * (4 * L + 1));
}
// After those, [L][G][TRACE_ALL] per layer and workgroup: qkv done, attention
// in, attention done, merge done, merge poll start (wall clock), merge poll
// count, loader 0's polls of a full ring, compute wave 0's polls for landed units.
constexpr int TRACE_ALL = 8;
__host__ __device__ constexpr int trace_words_all(int L, int G) { return trace_words(L) + L * G * TRACE_ALL; }
__device__ __forceinline__ int trace_slot(int wg, int G) {
    return wg == 0 ? 0 : wg == 1 ? 1 : wg == G / 2 ? 2 : wg == G - 1 ? 3 : -1;
}
enum { M_QKV = 0, M_O, M_GU, M_DOWN, M_LM };

enum : uint32_t { ERR_INPUT = 1, ERR_TIMEOUT_X = 2, ERR_TIMEOUT_LDS = 3 };

struct Smem {
    u32x4_t ring[RU * 64];    // weight units in flight to the compute waves (unit u in slot u % RU)
    bf16_t x[MAX_X];          // the current matrix's input vector
    float rows[MAX_ROWS];     // row sums of the current matrix (this workgroup's rows)
    bf16_t own[MAX_OWN];      // this workgroup's residual rows
    bf16_t kc[ATT_KEYS * PD]; // attention: K tiles (32 keys each, swizzled) of this workgroup's range
    bf16_t vc[ATT_KEYS * PD]; //            and the V tiles
    bf16_t qs[PGROUP * PD];   //            the 4 query heads, normed and rotated
    bf16_t knew[PD];          //            this token's K (normed, rotated) and V
    bf16_t vnew[PD];
    int pK[5], prb[5], pre[5];  // per streamed-matrix kind: K and this workgroup's rows [rb, re)
    int poff[5];              // per kind: first unit within a layer (LM: within the LM head)
    int ulayer;               // units per layer
    __align__(16) int landed[4];  // per loader wave: its units (every NLOAD-th) landed in the ring
    __align__(16) int prog[4];    // per compute wave: every unit of its below this index consumed
    int ready;                // matrices whose input is staged (control -> compute waves)
    int done;                 // 64 x (compute wave, matrix) completions (compute waves -> control)
    int abort;
};
static_assert(sizeof(Smem) <= LDS_BYTES, "LDS layout");
static_assert(NLOAD <= 4 && NCOMP == 4, "landed and prog are read as one 16-byte word");

struct PArgs {
    const q3_layer* layers;
    const bf16_t* embed;
    const bf16_t* final_norm;
    const bf16_t* lm_head;
    const bf16_t* cos_t;
    const bf16_t* sin_t;
    bf16_t* cache_k;
    bf16_t* cache_v;
    int64_t* tokens;
    int64_t* pos;
    bf16_t* logits;           // optional BF16 logits [V]
    uint32_t* state;          // [0] step epoch, [1] error code
    uint32_t* resid_x;        // [H] words
    uint32_t* qkv_x;          // [(Hq + 2 Hkv) * 128] words
    uint32_t* attn_x;         // [Hq * 128] words
    uint32_t* act_x;          // [I] words
    uint32_t* part_x;         // [Hkv * splits * 4 * PREC] words
    uint32_t* lm_x;           // [grid * 4] words
    uint64_t* trace;          // optional timestamps (q3_persist_trace_words() words), or NULL
    int L, H, I, V, Hq, Hkv, capacity;
    float eps, scale;
};

// The kernel's arguments, read in place from the kernarg segment (scalar loads)
// by every function: a by-value copy would be spilled to the stack for the
// noinline control-wave helpers.
typedef const __attribute__((address_space(4))) PArgs KArgs;
// The kernel takes the kernarg-segment pointer once and hands it down: the
// callable-function ABI passes no kernarg pointer, so the intrinsic is only
// valid in the kernel itself.  A pointer that arrives as a function argument
// sits in vector registers (divergent to the compiler); uni_ptr moves it back to
// scalar registers so loads through it are scalar loads.
__device__ __forceinline__ KArgs* uni_ptr(KArgs* p) {
    const uint64_t v = (uint64_t)p;
    const uint32_t lo = (uint32_t)__builtin_amdgcn_readfirstlane((int)(uint32_t)v);
    const uint32_t hi = (uint32_t)__builtin_amdgcn_readfirstlane((int)(uint32_t)(v >> 32));
    return (KArgs*)(((uint64_t)hi << 32) | lo);
}

// Layer l's pointer table, read through the constant address space (scalar
// loads): it is read-only for the whole launch, and a vector load of it would
// make the loaders wait for every weight load in flight.
typedef const __attribute__((address_space(4))) q3_layer KLayer;
__device__ __forceinline__ KLayer& layer(KArgs& a, int l) { return ((KLayer*)a.layers)[l]; }

// The workgroup's LDS (one workgroup per CU).  A file-scope __shared__ object,
// so helpers address it as LDS (ds_* instructions) rather than through generic
// pointers, which would also count on the vector-memory counter.
__shared__ __align__(16) Smem g_sm;

struct MatPart {
    int K, rb, re;
};

// floor(n * i / G); n * i < 2^31 for every caller (checked on the host).
__device__ __forceinline__ int part(int n, int i, int G) { return (int)((uint32_t)(n * i) / (uint32_t)G); }

// This workgroup's rows [rb, re) of streamed matrix kind m and its K.  gate/up
// rows are split in (gate, up) pairs so SwiGLU stays inside one workgroup.
__device__ __forceinline__ MatPart mat_part(KArgs& a, int m, int wg, int G) {
    const int qkv_rows = (a.Hq + 2 * a.Hkv) * PD;
    switch (m) {
        case M_QKV: return {a.H, part(qkv_rows, wg, G), part(qkv_rows, wg + 1, G)};
        case M_O: return {a.Hq * PD, part(a.H, wg, G), part(a.H, wg + 1, G)};
        case M_GU: return {a.H, 2 * part(a.I, wg, G), 2 * part(a.I, wg + 1, G)};
        case M_DOWN: return {a.I, part(a.H, wg, G), part(a.H, wg + 1, G)};
        default: return {a.H, part(a.V, wg, G), part(a.V, wg + 1, G)};
    }
}

// Streamed matrix mi of the step: 4 per layer (qkv, o, gate/up, down), then the LM head.
__device__ __forceinline__ int mat_kind(int mi, int L) { return mi == 4 * L ? M_LM : (mi & 3); }
__device__ __forceinline__ const bf16_t* mat_w(KArgs& a, int mi) {
    if (mi == 4 * a.L) return a.lm_head;
    KLayer& ly = layer(a, mi >> 2);
    switch (mi & 3) {
        case 0: return ly.qkv;
        case 1: return ly.o;
        case 2: return ly.gate_up;
        default: return ly.down;
    }
}

// ------------------------------------------------------- coherent exchange


// Loads through explicitly global pointers: pointers read from memory (the
// layer table) are otherwise generic, and generic (flat) loads also count on
// the LDS counter, so every LDS wait would drain the weight stream.
typedef __attribute__((address_space(1))) const u32x4_t* gvec;
typedef __attribute__((address_space(1))) u32x4_t* gvec_mut;
__device__ __forceinline__ u32x4_t ldg_nt(const void* p) { return __builtin_nontemporal_load((gvec)p); }
__device__ __forceinline__ u32x4_t ldg(const void* p) { return *(gvec)p; }
__device__ __forceinline__ void stg(void* p, u32x4_t v) { *(gvec_mut)p = v; }

__device__ __forceinline__ float dot8v(u32x4_t a, u32x4_t b, float c) {
    c = dot2(a.x, b.x, c);
    c = dot2(a.y, b.y, c);
    c = dot2(a.z, b.z, c);
    c = dot2(a.w, b.w, c);
    return c;
}

// Sum over the 16 lanes of each row (DPP), returned to every lane of the row.
__device__ __forceinline__ float row16_dpp(float v) {
    v += Q3_DPP(v, 0xb1);
    v += Q3_DPP(v, 0x4e);
    v += Q3_DPP(v, 0x124);
    v += Q3_DPP(v, 0x128);
    return v;
}

__device__ __forceinline__ bool better(float v, int i, float bv, int bi) {
    return v > bv || (v == bv && i < bi);
}

// ------------------------------------------------------ loaders and compute


__device__ __forceinline__ int lds_ready() {
    return uni(__hip_atomic_load(&g_sm.ready, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP));
}


__device__ __forceinline__ bool wait_ready(int mi) {
    SpinBound sb;
    while (lds_ready() <= mi) {
        __builtin_amdgcn_s_sleep(1);
        if (!sb.ok(STREAM_TIMEOUT)) {
            __hip_atomic_store(&g_sm.abort, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
            return false;
        }
    }
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
    return true;
}

// LDS accesses of the loader waves, as inline assembly: the compiler cannot
// tell them apart from the ring slots its own direct-to-LDS loads are writing,
// and would otherwise wait for every load in flight before each of them.
__device__ __forceinline__ uint32_t lds_addr(const void* p) {
    return (uint32_t)(uintptr_t)((const __attribute__((address_space(3))) void*)p);
}
__device__ __forceinline__ int lds_load_asm(const int* p) {
    int v;
    asm volatile("ds_read_b32 %0, %1\n\ts_waitcnt lgkmcnt(0)" : "=v"(v) : "v"(lds_addr(p)) : "memory");
    return uni(v);
}
// Four counters at once (16-byte aligned).
__device__ __forceinline__ u32x4_t lds_load4_asm(const int* p) {
    u32x4_t v;
    asm volatile("ds_read_b128 %0, %1\n\ts_waitcnt lgkmcnt(0)" : "=v"(v) : "v"(lds_addr(p)) : "memory");
    return v;
}
__device__ __forceinline__ void lds_store_asm(int* p, int v) {
    asm volatile("ds_write_b32 %0, %1" : : "v"(lds_addr(p)), "v"(v) : "memory");
}
// s_waitcnt vmcnt(n) with the other counters left open (gfx9 encoding).
#define Q3_WAIT_VM(n) __builtin_amdgcn_s_waitcnt(((n) & 15) | (((n) >> 4) << 14) | (7 << 4) | (15 << 8))

// s_waitcnt vmcnt(n) for a run-time n in [0, N].
template <int N>
__device__ __forceinline__ void wait_vm_le(int n) {
    if constexpr (N == 0) {
        Q3_WAIT_VM(0);
    } else {
        if (n >= N) {
            Q3_WAIT_VM(N);
            return;
        }
        wait_vm_le<N - 1>(n);
    }
}

// Weight units of this workgroup for the whole step, in order, into the LDS
// ring: loader w takes units w, w + NLOAD, ... of the step's stream (every
// matrix's rows [rb, re), each row's 512-element chunks in order).  A unit goes
// out once its slot's previous unit has been consumed (every compute wave's
// progress past it); the wave keeps LDEPTH loads in flight and publishes how
// many of its units have landed.  The row partition comes from the kernel
// arguments, not from LDS: after the first ring load, any LDS read the
// compiler sees would wait for every load in flight.
__device__ void loader(KArgs* ka, int w, int lane) {
    KArgs& a = *uni_ptr(ka);
    w = uni(w);
    const int last = 4 * a.L;
    int issued = 0;  // units issued
    int outs = 0;    // of those, possibly still in flight (the last `outs`)
    int minp = 0;    // cached min of the compute waves' progress
    auto min_prog = [&]() {
        const u32x4_t v = lds_load4_asm(g_sm.prog);
        return uni(min(min((int)v.x, (int)v.y), min((int)v.z, (int)v.w)));
    };
    // Trace (loader 0): polls of a full ring per layer, in the all-workgroup
    // trace; in the traced workgroups, when each matrix's first unit went out.
    uint64_t* tra = a.trace && w == 0 ? a.trace + trace_words(a.L) : nullptr;
    uint64_t* tri = nullptr;
    if (tra && trace_slot(blockIdx.x, gridDim.x) >= 0)
        tri = a.trace + (size_t)trace_slot(blockIdx.x, gridDim.x) * (trace_words(a.L) / TRACE_WGS) +
              (a.L + 1) * TRACE_EV + 2 * (4 * a.L + 1);
    int polls = 0;
    int u = 0;  // stream index of the current matrix's first unit
    for (int mi = 0; mi <= last; ++mi) {
        const MatPart mp = mat_part(a, mat_kind(mi, a.L), blockIdx.x, gridDim.x);
        const int kc = mp.K / CHUNK;
        const int n = uni((mp.re - mp.rb) * kc);
        const bf16_t* base = mat_w(a, mi) + (int64_t)mp.rb * mp.K + lane * 8;
        if (tri) tri[mi] = wall_clock64();
        for (int i = uni((w - u % NLOAD + NLOAD) % NLOAD); i < n; i += NLOAD) {
            const int gu = u + i;
            if (gu - RU >= minp) {
                // The slot still holds an unconsumed unit: while waiting,
                // publish this wave's loads one by one as they land (the
                // consumers may be waiting for exactly those).
                SpinBound sb;
                while (gu - RU >= (minp = min_prog())) {
                    ++polls;
                    if (outs > 0) {
                        --outs;
                        wait_vm_le<LDEPTH>(outs);
                        lds_store_asm(&g_sm.landed[w], issued - outs);
                        continue;
                    }
                    __builtin_amdgcn_s_sleep(1);
                    if (lds_load_asm(&g_sm.abort) || !sb.ok(STREAM_TIMEOUT)) {
                        lds_store_asm(&g_sm.abort, 1);
                        return;
                    }
                }
            }
            __builtin_amdgcn_global_load_lds((const __attribute__((address_space(1))) void*)(base + (int64_t)i * CHUNK),
                                             (__attribute__((address_space(3))) void*)&g_sm.ring[(gu % RU) * 64],
                                             16, 0, 2 /* non-temporal */);
            issued = uni(issued + 1);
            if (++outs > LDEPTH) {
                Q3_WAIT_VM(LDEPTH);
                outs = LDEPTH;
                lds_store_asm(&g_sm.landed[w], issued - LDEPTH);
            }
            outs = uni(outs);
        }
        u = uni(u + n);
        if (tra && (mi & 3) == 3 && mi < last) {
            tra[((size_t)(mi >> 2) * gridDim.x + blockIdx.x) * TRACE_ALL + 6] = polls;
            polls = 0;
        }
    }
    Q3_WAIT_VM(0);
    lds_store_asm(&g_sm.landed[w], issued);
}

// Every unit of the stream below the returned index has landed in the ring
// (loader w's first landed[w] units are w, w + NLOAD, ...).
__device__ __forceinline__ int landed_below() {
    const u32x4_t v = lds_load4_asm(g_sm.landed);
    const int n[4] = {(int)v.x, (int)v.y, (int)v.z, (int)v.w};
    int m = 0x7fffffff;
#pragma unroll
    for (int w = 0; w < NLOAD; ++w) m = min(m, w + NLOAD * n[w]);
    return uni(m);
}

// Compute wave c: for every matrix, once its input is staged, the dot products
// of rows rb + c, rb + c + NCOMP, ... with x.  A row is taken once all its
// units have landed; its chunks are read from the ring in order and summed per
// lane, then across the wave -- the arithmetic and order of the GEMV kernel
// (q3_gemv).  prog[c] then moves to the first unit of the wave's next row.
__device__ void compute(KArgs* ka, int c, int lane) {
    KArgs& a = *uni_ptr(ka);
    c = uni(c);
    const int last = 4 * a.L;
    const int ulayer = uni(g_sm.ulayer);
    int bound = 0;  // cached landed_below()
    uint64_t* tra = a.trace && c == 0 ? a.trace + trace_words(a.L) : nullptr;
    int polls = 0;  // trace: polls for landed units per layer (compute wave 0)
    uint64_t* tr = nullptr;  // compute wave 0's input waits, in the traced workgroups
    if (a.trace && c == 0 && trace_slot(blockIdx.x, gridDim.x) >= 0)
        tr = a.trace + (size_t)trace_slot(blockIdx.x, gridDim.x) * (trace_words(a.L) / TRACE_WGS) + (a.L + 1) * TRACE_EV;
    for (int mi = 0; mi <= last; ++mi) {
        if (tr) tr[2 * mi] = wall_clock64();
        if (!wait_ready(mi)) return;
        if (tr) tr[2 * mi + 1] = wall_clock64();
        const int kind = mat_kind(mi, a.L);
        const int K = uni(g_sm.pK[kind]), rb = uni(g_sm.prb[kind]), re = uni(g_sm.pre[kind]);
        const int kc = K / CHUNK;
        const int base = (mi == last ? a.L * ulayer : (mi >> 2) * ulayer) + uni(g_sm.poff[kind]);
        const int next = mi == last ? 0x7fffffff
                       : mi + 1 == last ? a.L * ulayer + uni(g_sm.poff[M_LM])
                       : ((mi + 1) >> 2) * ulayer + uni(g_sm.poff[mat_kind(mi + 1, a.L)]);
        for (int r = rb + c; r < re; r += NCOMP) {
            const int u0 = uni(base + (r - rb) * kc);
            if (bound < u0 + kc) {
                SpinBound sb;
                while ((bound = landed_below()) < u0 + kc) {
                    ++polls;
                    __builtin_amdgcn_s_sleep(1);
                    if (!sb.ok(STREAM_TIMEOUT)) {
                        __hip_atomic_store(&g_sm.abort, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
                        return;
                    }
                }
                __atomic_signal_fence(__ATOMIC_SEQ_CST);
            }
            float acc = 0.f;
            int slot = u0 % RU;
#pragma unroll 4
            for (int ch = 0; ch < kc; ++ch) {
                const u32x4_t wv = g_sm.ring[slot * 64 + lane];
                const u32x4_t xv = *reinterpret_cast<const u32x4_t*>(g_sm.x + ch * CHUNK + lane * 8);
                acc = dot8v(wv, xv, acc);
                slot = slot + 1 == RU ? 0 : slot + 1;
            }
            g_sm.rows[r - rb] = wave_sum(acc);  // every lane holds the sum: branch-free store
            __atomic_signal_fence(__ATOMIC_SEQ_CST);
            __hip_atomic_store(&g_sm.prog[c], r + NCOMP < re ? u0 + NCOMP * kc : next, __ATOMIC_RELAXED,
                               __HIP_MEMORY_SCOPE_WORKGROUP);
        }
        __atomic_signal_fence(__ATOMIC_SEQ_CST);
        __hip_atomic_store(&g_sm.prog[c], next, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
        // Every lane adds 1 (a uniform operand: one ds_add of 64, no loop over lanes).
        __hip_atomic_fetch_add(&g_sm.done, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
        if (tra && (mi & 3) == 3 && mi < last) {
            tra[((size_t)(mi >> 2) * gridDim.x + blockIdx.x) * TRACE_ALL + 7] = polls;
            polls = 0;
        }
    }
}

// ----------------------------------------------------------------- control

struct Ctl {
    KArgs* ka;
    uint64_t* tr;  // this workgroup's control-wave trace row, or NULL
    uint64_t* tra; // the all-workgroup trace, or NULL
    int lane, wg, G;
    int pos;
    int64_t tok;
    uint32_t fbase;
    int staged;

    // Arguments reach noinline helpers in vector registers; the wave-uniform
    // fields go back to scalar registers so branches on them stay scalar.
    __device__ void scalarize() {
        ka = uni_ptr(ka);
        wg = uni(wg);
        G = uni(G);
        pos = uni(pos);
        fbase = (uint32_t)uni((int)fbase);
        staged = uni(staged);
    }

    __device__ void mark(int l, int ev) const {
        if (tr && lane == 0) tr[l * TRACE_EV + ev] = wall_clock64();
    }
    __device__ void mark_all(int l, int ev) const {
        if (tra && lane == 0) tra[((size_t)l * G + wg) * TRACE_ALL + ev] = wall_clock64();
    }

    __device__ uint32_t flag(int l, int op) const {
        uint32_t i = fbase + (uint32_t)(l * OP_COUNT + op);
        if (i >= 65535u) i -= 65535u;
        return i + 1u;
    }
};

// Ctl as scalar arguments of the noinline helpers: a struct argument would be
// passed through scratch memory, and every call would wait for it.
#define Q3_CTL_PARAMS                                                                                  \
    KArgs *c_ka, uint64_t *c_tr, uint64_t *c_tra, int c_lane, int c_wg, int c_G, int c_pos, int64_t c_tok, \
        uint32_t c_fbase, int c_staged
#define Q3_CTL_ARGS(c) (c).ka, (c).tr, (c).tra, (c).lane, (c).wg, (c).G, (c).pos, (c).tok, (c).fbase, (c).staged
#define Q3_CTL_MAKE                                                                \
    Ctl c{c_ka, c_tr, c_tra, c_lane, c_wg, c_G, c_pos, c_tok, c_fbase, c_staged}; \
    c.scalarize()

__device__ void fail(Ctl& c, uint32_t code) {
    __hip_atomic_store(c.ka->state + 1, code, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    if (c.lane == 0) c.ka->tokens[0] = -1;
    __hip_atomic_store(&g_sm.abort, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
    __hip_atomic_store(&g_sm.ready, 1 << 30, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
}

__device__ __forceinline__ void publish(Ctl& c) {
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
    __hip_atomic_store(&g_sm.ready, ++c.staged, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
}

__device__ bool wait_done(Ctl& c) {
    const int target = c.staged * NCOMP * Q3_WAVE;  // each compute wave adds 64 per matrix
    auto done = []() { return uni(__hip_atomic_load(&g_sm.done, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP)); };
    SpinBound sb;
    while (done() < target) {
        __builtin_amdgcn_s_sleep(1);
        if (uni(__hip_atomic_load(&g_sm.abort, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP)) ||
            !sb.ok(CTL_TIMEOUT)) {
            fail(c, ERR_TIMEOUT_LDS);
            return false;
        }
    }
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
    return true;
}


// Bounded wait helper for the control wave's polls: false once the wait has
// run past CTL_TIMEOUT (after recording the failure).
struct Deadline {
    SpinBound sb;
    __device__ bool tick(Ctl& c) {
        if (!sb.ok(CTL_TIMEOUT)) {
            fail(c, ERR_TIMEOUT_X);
            return false;
        }
        __builtin_amdgcn_s_sleep(1);
        return true;
    }
};

// Gather flagged words [n8 chunks of 8 words]: lane l takes chunks l + 64 m for
// m in [m0, m0 + MC) (the last partial row of chunks re-reads chunk n8 - 1),
// re-reading them all until every word carries flag F.
template <int MC>
__device__ bool poll_chunks(Ctl& c, const uint32_t* base, int n8, int m0, uint32_t F, u32x4_t (&lo)[MC],
                            u32x4_t (&hi)[MC]) {
    const auto rs = rsrc(base);
    const int per = min(MC, (n8 + 63) / 64 - m0);  // wave-uniform
    const uint32_t Fs = F << 16;
    Deadline dl;
    for (;;) {
#pragma unroll
        for (int m = 0; m < MC; ++m)
            if (m < per) {
                const int off = min(c.lane + 64 * (m0 + m), n8 - 1) * 32;
                lo[m] = ld_coh(rs, off);
                hi[m] = ld_coh(rs, off + 16);
            }
        uint32_t bad = 0;
#pragma unroll
        for (int m = 0; m < MC; ++m)
            if (m < per) bad |= unflagged(lo[m], Fs) | unflagged(hi[m], Fs);
        if (__all(bad == 0)) break;
        if (!dl.tick(c)) return false;
    }
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
    return true;
}

// x = RMSNorm(src) * gain into LDS, K <= 4096.  src is the flagged residual, or
// (layer 0) the embedding row.  The sum of squares follows the GEMV prologue
// (q3_gemv stage_x): a 256-thread block where thread t sums chunks t, t + 256,
// then each 64-thread wave is reduced and the four wave sums are added as
// (w0 + w1) + (w2 + w3).  Lane l plays threads l, l+64, l+128, l+192: its chunk
// l + 64 m belongs to thread l + 64 (m % 4).
__device__ __attribute__((noinline)) bool stage_norm(Q3_CTL_PARAMS, const uint32_t* src_x, uint32_t F, const bf16_t* src_plain,
                           const bf16_t* gain, int K) {
    Q3_CTL_MAKE;
    constexpr int MC = 8;
    const int n8 = K / 8;
    // The gain does not depend on the exchange: its loads go out first.
    uint4 gv[MC];
#pragma unroll
    for (int m = 0; m < MC; ++m)
        if (c.lane + 64 * m < n8) {
            const u32x4_t t = ldg(gain + (c.lane + 64 * m) * 8);
            gv[m] = make_uint4(t.x, t.y, t.z, t.w);
        }
    uint4 xv[MC];
    if (src_plain) {
#pragma unroll
        for (int m = 0; m < MC; ++m)
            if (c.lane + 64 * m < n8) {
                const u32x4_t t = ldg(src_plain + (c.lane + 64 * m) * 8);
                xv[m] = make_uint4(t.x, t.y, t.z, t.w);
            }
    } else {
        u32x4_t lo[MC], hi[MC];
        if (!poll_chunks<MC>(c, src_x, n8, 0, F, lo, hi)) return false;
#pragma unroll
        for (int m = 0; m < MC; ++m)
            xv[m] = make_uint4(bfpair(lo[m].x, lo[m].y), bfpair(lo[m].z, lo[m].w), bfpair(hi[m].x, hi[m].y),
                               bfpair(hi[m].z, hi[m].w));
    }
    float ss[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int m = 0; m < MC; ++m) {
        if (c.lane + 64 * m < n8) {
            const uint4 v = xv[m];
            float s = ss[m & 3];
            s += bflo(v.x) * bflo(v.x); s += bfhi(v.x) * bfhi(v.x);
            s += bflo(v.y) * bflo(v.y); s += bfhi(v.y) * bfhi(v.y);
            s += bflo(v.z) * bflo(v.z); s += bfhi(v.z) * bfhi(v.z);
            s += bflo(v.w) * bflo(v.w); s += bfhi(v.w) * bfhi(v.w);
            ss[m & 3] = s;
        }
    }
    const float total = (wave_sum(ss[0]) + wave_sum(ss[1])) + (wave_sum(ss[2]) + wave_sum(ss[3]));
    const float inv = inv_rms(total, K, c.ka->eps);
#pragma unroll
    for (int m = 0; m < MC; ++m) {
        if (c.lane + 64 * m < n8) {
            uint4 v = xv[m];
            const uint4 g = gv[m];
            v.x = pack2(norm_elem(bflo(v.x), inv, bflo(g.x)), norm_elem(bfhi(v.x), inv, bfhi(g.x)));
            v.y = pack2(norm_elem(bflo(v.y), inv, bflo(g.y)), norm_elem(bfhi(v.y), inv, bfhi(g.y)));
            v.z = pack2(norm_elem(bflo(v.z), inv, bflo(g.z)), norm_elem(bfhi(v.z), inv, bfhi(g.z)));
            v.w = pack2(norm_elem(bflo(v.w), inv, bflo(g.w)), norm_elem(bfhi(v.w), inv, bfhi(g.w)));
            *reinterpret_cast<uint4*>(g_sm.x + (c.lane + 64 * m) * 8) = v;
        }
    }
    return true;
}

// x = the flagged vector src (K elements) into LDS as BF16.
__device__ __attribute__((noinline)) bool stage_plain(Q3_CTL_PARAMS, const uint32_t* src_x, uint32_t F, int K) {
    Q3_CTL_MAKE;
    const int n8 = K / 8;
    for (int m0 = 0; 64 * m0 < n8; m0 += STAGE_CHUNKS) {
        u32x4_t lo[STAGE_CHUNKS], hi[STAGE_CHUNKS];
        if (!poll_chunks<STAGE_CHUNKS>(c, src_x, n8, m0, F, lo, hi)) return false;
#pragma unroll
        for (int m = 0; m < STAGE_CHUNKS; ++m) {
            const int ch = c.lane + 64 * (m0 + m);
            if (ch < n8)
                *reinterpret_cast<uint4*>(g_sm.x + ch * 8) =
                    make_uint4(bfpair(lo[m].x, lo[m].y), bfpair(lo[m].z, lo[m].w), bfpair(hi[m].x, hi[m].y),
                               bfpair(hi[m].z, hi[m].w));
        }
    }
    return true;
}

// ----------------------------------------------------------- attention unit

// Keys [base, base + ATT_KEYS) of one KV head into the two LDS tiles, all loads
// issued before any wait.  Load j moves keys 4j..4j+3 of the pair (tile j / 8):
// lane l takes chunk (l % 16) ^ (key & 15) of key 4 j + l / 16, which is its
// slot in the tile's swizzled layout (q3attn::kv_slot).  Rows past `last`
// re-read row `last` (masked later); the new token's row is substituted later.
__device__ __attribute__((noinline)) void gather_kv(const bf16_t* kb, const bf16_t* vb, int base, int last,
                                                   int lane) {
    constexpr int NL = ATT_KEYS / 4;
    u32x4_t k[NL], v[NL];
#pragma unroll
    for (int j = 0; j < NL; ++j) {
        const int r = 4 * j + (lane >> 4);
        const int c = (lane & 15) ^ (r & 15);
        const int64_t off = (int64_t)min(base + r, last) * PD + c * 8;
        k[j] = ldg(kb + off);
        v[j] = ldg(vb + off);
    }
#pragma unroll
    for (int j = 0; j < NL; ++j) {
        reinterpret_cast<u32x4_t*>(g_sm.kc)[64 * j + lane] = k[j];
        reinterpret_cast<u32x4_t*>(g_sm.vc)[64 * j + lane] = v[j];
    }
}

// Per-head RMSNorm + RoPE of a 128-wide row spread over the 16 lanes of each
// lane row (lane holds dims 8 (l % 16) .. +8; dims d and d + 64 are 8 lanes
// apart); g, cv, sv are this lane's 8 gains, cosines and sines.  t = bf16(x * rsqrt(mean(x^2) + eps)); y = bf16(w * t); then
// lo' = bf16(bf16(lo c) + bf16(-hi s)), hi' = bf16(bf16(hi c) + bf16(lo s))
// (reference fused.py:196-219, engine.py:91-109).
__device__ __forceinline__ u32x4_t norm_rope8(u32x4_t x, u32x4_t g, u32x4_t cv, u32x4_t sv, float eps, int lane) {
    const int d0 = (lane & 15) * 8;
    float f[8] = {bflo(x.x), bfhi(x.x), bflo(x.y), bfhi(x.y), bflo(x.z), bfhi(x.z), bflo(x.w), bfhi(x.w)};
    float ss = 0.f;
#pragma unroll
    for (int e = 0; e < 8; ++e) ss += f[e] * f[e];
    const float inv = inv_rms(row16_dpp(ss), PD, eps);
    const float gf[8] = {bflo(g.x), bfhi(g.x), bflo(g.y), bfhi(g.y), bflo(g.z), bfhi(g.z), bflo(g.w), bfhi(g.w)};
    float n[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) n[e] = bf2f(norm_elem(f[e], inv, gf[e]));
    const float cf[8] = {bflo(cv.x), bfhi(cv.x), bflo(cv.y), bfhi(cv.y), bflo(cv.z), bfhi(cv.z), bflo(cv.w), bfhi(cv.w)};
    const float sf[8] = {bflo(sv.x), bfhi(sv.x), bflo(sv.y), bfhi(sv.y), bflo(sv.z), bfhi(sv.z), bflo(sv.w), bfhi(sv.w)};
    const bool low = (lane & 8) == 0;  // dims < 64
    uint32_t o[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) {
        const float partner = __shfl_xor(n[e], 8, Q3_WAVE);
        o[e] = low ? f2bf(rbf(n[e] * cf[e]) + rbf(-partner * sf[e]))
                   : f2bf(rbf(n[e] * cf[e]) + rbf(partner * sf[e]));
    }
    u32x4_t r;
    r.x = pack2(o[0], o[1]);
    r.y = pack2(o[2], o[3]);
    r.z = pack2(o[4], o[5]);
    r.w = pack2(o[6], o[7]);
    return r;
}

struct AttnPlan {
    int h, s, S;          // KV head, key range, ranges per head
    int k0, k1;           // keys [k0, k1) (the new token's key pos included by the owner)
    bool owner;           // this range ends at the new token (pos)
    const bf16_t* kb;
    const bf16_t* vb;
};

__device__ AttnPlan attn_plan(const Ctl& c, int l) {
    KArgs& a = *c.ka;
    AttnPlan p;
    p.S = c.G / a.Hkv;
    p.h = c.wg % a.Hkv;
    p.s = c.wg / a.Hkv;
    const int ctx = c.pos + 1;
    const int per = (ctx + p.S - 1) / p.S;
    p.k0 = p.s * per;
    p.k1 = min(p.k0 + per, ctx);
    p.owner = p.k0 <= c.pos && c.pos < p.k1;
    const int64_t head = ((int64_t)l * a.Hkv + p.h) * a.capacity * PD;  // cache [L, 1, Hkv, C, 128]
    p.kb = a.cache_k + head;
    p.vb = a.cache_v + head;
    return p;
}

// One (KV head, key range) unit: this layer's q / k / v rows of the head from
// the exchange, q and k normed and rotated, the new token's K and V appended to
// the cache by the range that holds it, then the online softmax over the cached
// keys (first set prefetched by the caller) and the new key.  Publishes the
// unnormalised partial (acc, m, l) of each of the 4 query heads.
__device__ __attribute__((noinline)) bool attention(Q3_CTL_PARAMS, int l, int p_h, int p_s, int p_S, int p_k0, int p_k1, bool p_owner,
                                                    const bf16_t* p_kb, const bf16_t* p_vb) {
    Q3_CTL_MAKE;
    const AttnPlan p{uni(p_h), uni(p_s), uni(p_S), uni(p_k0), uni(p_k1), uni(p_owner ? 1 : 0) != 0, p_kb, p_vb};
    KArgs& a = *c.ka;
    const int lane = c.lane, g = lane >> 4, d0 = (lane & 15) * 8;
    const int qsz = a.Hq * PD;
    // q rows of heads 4h..4h+3 (one per lane row), then the k and v rows (every lane row).
    const auto rs = rsrc(a.qkv_x);
    const int qoff = ((p.h * PGROUP + g) * PD + d0) * 4;
    const int koff = (qsz + p.h * PD + d0) * 4;
    const int voff = (qsz + a.Hkv * PD + p.h * PD + d0) * 4;
    const uint32_t F = c.flag(l, OP_QKV);
    // The gains and this position's cos / sin do not depend on the exchange:
    // their loads go out first and land while the q / k / v rows are awaited.
    KLayer& ly = layer(a, l);
    const bf16_t* cosr = a.cos_t + (int64_t)c.pos * PD;
    const bf16_t* sinr = a.sin_t + (int64_t)c.pos * PD;
    const u32x4_t gq = ldg(ly.q_norm + d0), gk = ldg(ly.k_norm + d0);
    const u32x4_t cv = ldg(cosr + d0), sv = ldg(sinr + d0);
    u32x4_t w[6];
    const uint32_t Fs = F << 16;
    Deadline dl;
    for (;;) {
        w[0] = ld_coh(rs, qoff); w[1] = ld_coh(rs, qoff + 16);
        w[2] = ld_coh(rs, koff); w[3] = ld_coh(rs, koff + 16);
        w[4] = ld_coh(rs, voff); w[5] = ld_coh(rs, voff + 16);
        uint32_t bad = 0;
#pragma unroll
        for (int i = 0; i < 6; ++i) bad |= unflagged(w[i], Fs);
        if (__all(bad == 0)) break;
        if (!dl.tick(c)) return false;
    }
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
    c.mark(l, T_ATT_IN);
    c.mark_all(l, 1);
    u32x4_t qv, kn, vn;
    qv.x = bfpair(w[0].x, w[0].y); qv.y = bfpair(w[0].z, w[0].w);
    qv.z = bfpair(w[1].x, w[1].y); qv.w = bfpair(w[1].z, w[1].w);
    kn.x = bfpair(w[2].x, w[2].y); kn.y = bfpair(w[2].z, w[2].w);
    kn.z = bfpair(w[3].x, w[3].y); kn.w = bfpair(w[3].z, w[3].w);
    vn.x = bfpair(w[4].x, w[4].y); vn.y = bfpair(w[4].z, w[4].w);
    vn.z = bfpair(w[5].x, w[5].y); vn.w = bfpair(w[5].z, w[5].w);
    const u32x4_t qr = norm_rope8(qv, gq, cv, sv, a.eps, lane);
    kn = norm_rope8(kn, gk, cv, sv, a.eps, lane);
    if (p.owner && g == 0) {
        // This token's K and V into the cache (fused.py:553-617); later steps read them.
        const int64_t off = (int64_t)c.pos * PD + d0;
        stg(const_cast<bf16_t*>(p.kb) + off, kn);
        stg(const_cast<bf16_t*>(p.vb) + off, vn);
    }
    // q of the 4 heads and the new K / V into LDS for the MFMA operands.
    reinterpret_cast<u32x4_t*>(g_sm.qs)[lane] = qr;
    if (g == 0) {
        reinterpret_cast<u32x4_t*>(g_sm.knew)[lane] = kn;
        reinterpret_cast<u32x4_t*>(g_sm.vnew)[lane] = vn;
    }
    const int n = lane & 15;
    q3attn::WaveState st;
#pragma unroll
    for (int kk = 0; kk < 4; ++kk) {
        u32x4_t v = u32x4_t{0u, 0u, 0u, 0u};
        if (n < PGROUP) v = reinterpret_cast<const u32x4_t*>(g_sm.qs)[(n * PD + 32 * kk + 8 * g) / 8];
        st.qb[kk] = __builtin_bit_cast(bf16x8_t, v);
    }
    st.m = -INFINITY;
    st.l = 0.f;
#pragma unroll
    for (int dm = 0; dm < 8; ++dm) st.acc[dm] = f32x4_t{0.f, 0.f, 0.f, 0.f};
    // The first two blocks were gathered while the projection streamed; longer
    // ranges gather two more blocks per round trip.
    for (int blk = p.k0; blk < p.k1; blk += q3attn::ABLK) {
        const int rel = blk - p.k0;
        if (rel != 0 && rel % ATT_KEYS == 0) gather_kv(p.kb, p.vb, blk, p.k1 - 1, lane);
        bf16_t* kt = g_sm.kc + ((rel / q3attn::ABLK) & 1) * q3attn::ABLK * PD;
        bf16_t* vt = g_sm.vc + ((rel / q3attn::ABLK) & 1) * q3attn::ABLK * PD;
        const int sub = (p.owner && blk <= c.pos && c.pos < blk + q3attn::ABLK) ? c.pos - blk : -1;
        q3attn::decode_block_tiles(st, kt, vt, blk, p.k1, sub, g_sm.knew, g_sm.vnew, a.scale, lane);
    }

    // Publish query head n's partial from lanes n < 4: O^T[16 dm + 4 g + i][n]
    // (unnormalised) and (m, l).
    const uint32_t FA = c.flag(l, OP_ATTN);
    if (n < PGROUP) {
        const auto ws = rsrc(a.part_x);
        const int rec = ((p.h * p.S + p.s) * PGROUP + n) * PREC * 4;  // bytes
#pragma unroll
        for (int dm = 0; dm < 8; ++dm) {
            const int w0 = 2 * (16 * dm + 4 * g) + rec / 4;
            u32x4_t o0, o1;
            o0.x = fhi(st.acc[dm][0], FA); o0.y = flo(st.acc[dm][0], FA);
            o0.z = fhi(st.acc[dm][1], FA); o0.w = flo(st.acc[dm][1], FA);
            o1.x = fhi(st.acc[dm][2], FA); o1.y = flo(st.acc[dm][2], FA);
            o1.z = fhi(st.acc[dm][3], FA); o1.w = flo(st.acc[dm][3], FA);
            st_coh(ws, w0 * 4, o0);
            st_coh(ws, w0 * 4 + 16, o1);
        }
        if (g == 0) {
            u32x4_t o;
            o.x = fhi(st.m, FA); o.y = flo(st.m, FA); o.z = fhi(st.l, FA); o.w = flo(st.l, FA);
            st_coh(ws, rec + 256 * 4, o);
        }
    }
    return true;
}

// This workgroup's slice of the split merge: outputs [o0, o0 + n) of the Hq*128
// attention vector (one query head), out = bf16(sum_s acc_s e^(m_s - M) /
// sum_s l_s e^(m_s - M)) over the key ranges that hold keys (fused.py:793-823).
__device__ __attribute__((noinline)) bool merge(Q3_CTL_PARAMS, int l) {
    Q3_CTL_MAKE;
    KArgs& a = *c.ka;
    const int lane = c.lane;
    const int T = a.Hq * PD;
    const int S = c.G / a.Hkv;
    const int o0 = part(T, c.wg, c.G), n = part(T, c.wg + 1, c.G) - o0;
    const int qh = o0 / PD, d0 = o0 % PD;
    const int h = qh / PGROUP, j = qh % PGROUP;
    const int ctx = c.pos + 1;
    const int per = (ctx + S - 1) / S;
    const int used = (ctx + per - 1) / per;  // ranges with keys
    const uint32_t F = c.flag(l, OP_ATTN);
    // Lane t reads ranges t and t + 64: (m, l) and acc[d0 .. d0 + n), n <= MAX_SLICE floats.
    constexpr int NQ = MAX_SLICE * 2 / 4;  // 16-byte pieces of acc per range
    u32x4_t accw[2][NQ], mlw[2];
    const int nq = (n * 2 + 3) / 4;
    const int nu = used > 64 ? 2 : 1;  // wave-uniform
    const uint32_t Fs = F << 16;
    Deadline dl;
    c.mark_all(l, 4);
    int iters = 0;
    for (;;) {
        ++iters;
        uint32_t bad = 0;
        const auto rs = rsrc(a.part_x);
#pragma unroll
        for (int u = 0; u < 2; ++u) {
            if (u < nu) {
                const int sidx = min(lane + 64 * u, used - 1);
                const int rec = ((h * S + sidx) * PGROUP + j) * PREC * 4;  // bytes
                mlw[u] = ld_coh(rs, rec + 256 * 4);
#pragma unroll
                for (int q = 0; q < NQ; ++q)
                    if (q < nq) accw[u][q] = ld_coh(rs, rec + (d0 * 2 + 4 * q) * 4);
            }
        }
#pragma unroll
        for (int u = 0; u < 2; ++u) {
            if (u < nu) {
                bad |= unflagged(mlw[u], Fs);
#pragma unroll
                for (int q = 0; q < NQ; ++q)
                    if (q < nq) bad |= unflagged(accw[u][q], Fs);
            }
        }
        if (__all(bad == 0)) break;
        if (!dl.tick(c)) return false;
    }
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
    c.mark(l, T_MRG_IN);
    if (c.tra && c.lane == 0) c.tra[((size_t)l * c.G + c.wg) * TRACE_ALL + 5] = iters;
    float ms[2], ls[2];
#pragma unroll
    for (int u = 0; u < 2; ++u) {
        const bool has = u < nu && lane + 64 * u < used;
        ms[u] = has ? funpack(mlw[u].x, mlw[u].y) : -INFINITY;
        ls[u] = has ? funpack(mlw[u].z, mlw[u].w) : 0.f;
    }
    const float M = wave_max(fmaxf(ms[0], ms[1]));
    float wt[2];
#pragma unroll
    for (int u = 0; u < 2; ++u) wt[u] = ms[u] == -INFINITY ? 0.f : expf(ms[u] - M);
    const float Ls = wave_sum(ls[0] * wt[0] + ls[1] * wt[1]);
    uint32_t mine = 0;
    const uint32_t FM = c.flag(l, OP_MERGE);
#pragma unroll
    for (int q = 0; q < NQ; ++q) {
        if (q < nq) {
#pragma unroll
            for (int e = 0; e < 2; ++e) {
                const int idx = 2 * q + e;  // output d0 + idx
                if (idx < n) {
                    float v = 0.f;
#pragma unroll
                    for (int u = 0; u < 2; ++u) {
                        const u32x4_t w = accw[u][q];
                        const float f = e == 0 ? funpack(w.x, w.y) : funpack(w.z, w.w);
                        v += (u < nu && lane + 64 * u < used) ? f * wt[u] : 0.f;
                    }
                    const float tot = wave_sum(v);
                    if (lane == idx) mine = f2bf(Ls > 0.f ? tot / Ls : 0.f);
                }
            }
        }
    }
    if (lane < n) st_coh32(a.attn_x + o0 + lane, word(mine, FM));
    return true;
}

// ------------------------------------------------------------- epilogues

__device__ __attribute__((noinline)) void publish_rows(Q3_CTL_PARAMS, uint32_t* dst, int rb, int n, uint32_t F) {
    Q3_CTL_MAKE;
    for (int i = c.lane; i < n; i += 64) st_coh32(dst + rb + i, word(f2bf(g_sm.rows[i]), F));
}

// resid = bf16(resid + bf16(row sum)) on this workgroup's residual rows (fused.py:135-138).
__device__ __attribute__((noinline)) void publish_resid(Q3_CTL_PARAMS, int rb, int n, uint32_t F) {
    Q3_CTL_MAKE;
    for (int i = c.lane; i < n; i += 64) {
        const uint32_t v = f2bf(bf2f(g_sm.own[i]) + rbf(g_sm.rows[i]));
        g_sm.own[i] = (bf16_t)v;
        st_coh32(c.ka->resid_x + rb + i, word(v, F));
    }
}

// act[j] = bf16(bf16(silu(g)) * u) from the interleaved rows (gate_j, up_j) (fused.py:107-111).
__device__ __attribute__((noinline)) void publish_swiglu(Q3_CTL_PARAMS, int rb, int n, uint32_t F) {
    Q3_CTL_MAKE;
    const int pb = rb / 2;
    for (int j = c.lane; j < n / 2; j += 64) {
        const float gte = rbf(g_sm.rows[2 * j]), up = rbf(g_sm.rows[2 * j + 1]);
        st_coh32(c.ka->act_x + pb + j, word(f2bf(silu_bf16(gte) * up), F));
    }
}

// (max BF16 logit, lowest index) of this workgroup's LM-head rows (engine.py:833).
__device__ __attribute__((noinline)) void publish_argmax(Q3_CTL_PARAMS, int rb, int n, uint32_t F) {
    Q3_CTL_MAKE;
    float bv = -INFINITY;
    int bi = 0x7fffffff;
    for (int i = c.lane; i < n; i += 64) {
        const uint32_t b = f2bf(g_sm.rows[i]);
        if (c.ka->logits) c.ka->logits[rb + i] = (bf16_t)b;
        const float v = bf2f(b);
        if (better(v, rb + i, bv, bi)) { bv = v; bi = rb + i; }
    }
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) {
        const float v = __shfl_xor(bv, o, Q3_WAVE);
        const int i = __shfl_xor(bi, o, Q3_WAVE);
        if (better(v, i, bv, bi)) { bv = v; bi = i; }
    }
    if (c.lane == 0) {
        u32x4_t o;
        o.x = fhi(bv, F); o.y = flo(bv, F);
        o.z = word((uint32_t)bi >> 16, F); o.w = word((uint32_t)bi & 0xffffu, F);
        st_coh(rsrc(c.ka->lm_x), c.wg * 16, o);
    }
}

// Workgroup 0: the greedy token from every workgroup's partial; advances pos and the epoch.
__device__ __attribute__((noinline)) bool finish(Q3_CTL_PARAMS, uint32_t epoch) {
    Q3_CTL_MAKE;
    const uint32_t F = c.flag(c.ka->L, 0);
    const auto rs = rsrc(c.ka->lm_x);
    float bv = -INFINITY;
    int bi = 0x7fffffff;
    for (int p0 = 0; p0 < c.G; p0 += 64) {
        const int p = p0 + c.lane;
        u32x4_t v;
        Deadline dl;
        for (;;) {
            v = ld_coh(rs, min(p, c.G - 1) * 16);
            if (__all(unflagged(v, F << 16) == 0)) break;
            if (!dl.tick(c)) return false;
        }
        if (p < c.G) {
            const float val = funpack(v.x, v.y);
            const int idx = (int)(((v.z & 0xffffu) << 16) | (v.w & 0xffffu));
            if (better(val, idx, bv, bi)) { bv = val; bi = idx; }
        }
    }
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) {
        const float v = __shfl_xor(bv, o, Q3_WAVE);
        const int i = __shfl_xor(bi, o, Q3_WAVE);
        if (better(v, i, bv, bi)) { bv = v; bi = i; }
    }
    if (c.lane == 0) {
        c.ka->tokens[0] = bi;
        c.ka->pos[0] = c.pos + 1;
        __hip_atomic_store(c.ka->state, epoch + 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    return true;
}

__device__ void control(KArgs* ka, int lane, int wg, int G) {
    ka = uni_ptr(ka);
    KArgs& a = *ka;
    Ctl c{ka, nullptr, nullptr, lane, uni(wg), uni(G), 0, 0, 0u, 0};
    {
        const int ts = trace_slot(c.wg, c.G);
        if (a.trace && ts >= 0) c.tr = a.trace + (size_t)ts * (trace_words(a.L) / TRACE_WGS);
        if (a.trace) c.tra = a.trace + trace_words(a.L);
    }
    c.mark(0, T_START);
    const uint32_t epoch = __hip_atomic_load(a.state, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    c.fbase = (uint32_t)(((uint64_t)epoch * (uint64_t)(a.L + 1) * OP_COUNT) % 65535u);
    const int64_t pos = a.pos[0], tok = a.tokens[0];
    if (pos < 0 || pos >= a.capacity || tok < 0 || tok >= a.V) {
        fail(c, ERR_INPUT);
        return;
    }
    c.pos = (int)pos;
    c.tok = tok;
    const MatPart pq = mat_part(a, M_QKV, c.wg, c.G), po = mat_part(a, M_O, c.wg, c.G);
    const MatPart pg = mat_part(a, M_GU, c.wg, c.G), pd = mat_part(a, M_DOWN, c.wg, c.G);
    const bf16_t* emb = a.embed + tok * a.H;
    for (int i = lane; i < po.re - po.rb; i += 64) g_sm.own[i] = emb[po.rb + i];

    for (int l = 0; l < a.L; ++l) {
        KLayer& ly = layer(a, l);
        // qkv = W_qkv . RMSNorm(resid)
        const bool ok = l == 0 ? stage_norm(Q3_CTL_ARGS(c), nullptr, 0, emb, ly.in_ln, a.H)
                               : stage_norm(Q3_CTL_ARGS(c), a.resid_x, c.flag(l - 1, OP_DOWN), nullptr, ly.in_ln, a.H);
        if (!ok) return;
        c.mark(l, T_QKV_IN);
        publish(c);
        // This layer's cached keys go out while the projection streams.
        const AttnPlan ap = attn_plan(c, l);
        if (ap.k0 < ap.k1) gather_kv(ap.kb, ap.vb, ap.k0, ap.k1 - 1, lane);
        if (!wait_done(c)) return;
        c.mark(l, T_QKV_DONE);
        c.mark_all(l, 0);
        publish_rows(Q3_CTL_ARGS(c), a.qkv_x, pq.rb, pq.re - pq.rb, c.flag(l, OP_QKV));
        if (!attention(Q3_CTL_ARGS(c), l, ap.h, ap.s, ap.S, ap.k0, ap.k1, ap.owner, ap.kb, ap.vb)) return;
        c.mark(l, T_ATT_DONE);
        c.mark_all(l, 2);
        if (!merge(Q3_CTL_ARGS(c), l)) return;
        c.mark(l, T_MRG_DONE);
        c.mark_all(l, 3);
        // resid += W_o . attn
        if (!stage_plain(Q3_CTL_ARGS(c), a.attn_x, c.flag(l, OP_MERGE), a.Hq * PD)) return;
        c.mark(l, T_O_IN);
        publish(c);
        if (!wait_done(c)) return;
        c.mark(l, T_O_DONE);
        publish_resid(Q3_CTL_ARGS(c), po.rb, po.re - po.rb, c.flag(l, OP_O));
        // act = SwiGLU(W_gu . RMSNorm(resid))
        if (!stage_norm(Q3_CTL_ARGS(c), a.resid_x, c.flag(l, OP_O), nullptr, ly.post_ln, a.H)) return;
        c.mark(l, T_GU_IN);
        publish(c);
        if (!wait_done(c)) return;
        c.mark(l, T_GU_DONE);
        publish_swiglu(Q3_CTL_ARGS(c), pg.rb, pg.re - pg.rb, c.flag(l, OP_GU));
        // resid += W_down . act
        if (!stage_plain(Q3_CTL_ARGS(c), a.act_x, c.flag(l, OP_GU), a.I)) return;
        c.mark(l, T_DN_IN);
        publish(c);
        if (!wait_done(c)) return;
        c.mark(l, T_DN_DONE);
        publish_resid(Q3_CTL_ARGS(c), pd.rb, pd.re - pd.rb, c.flag(l, OP_DOWN));
    }
    // token = argmax(E . RMSNorm(resid))
    if (!stage_norm(Q3_CTL_ARGS(c), a.resid_x, c.flag(a.L - 1, OP_DOWN), nullptr, a.final_norm, a.H)) return;
    c.mark(a.L, T_QKV_IN);
    publish(c);
    if (!wait_done(c)) return;
    c.mark(a.L, T_QKV_DONE);
    const MatPart pl = mat_part(a, M_LM, c.wg, c.G);
    publish_argmax(Q3_CTL_ARGS(c), pl.rb, pl.re - pl.rb, c.flag(a.L, 0));
    if (wg == 0) finish(Q3_CTL_ARGS(c), epoch);
}

__global__ __launch_bounds__(PTHREADS) void decode_persist_kernel(PArgs args) {
    (void)args;  // read in place through the kernarg segment
    KArgs* ka = (KArgs*)(__builtin_amdgcn_kernarg_segment_ptr());
    const int wave = uni(threadIdx.x >> 6), lane = threadIdx.x & 63;
    if (threadIdx.x == 0) {
        int off = 0;
        for (int k = 0; k < 5; ++k) {
            const MatPart p = mat_part(*ka, k, blockIdx.x, gridDim.x);
            g_sm.pK[k] = p.K;
            g_sm.prb[k] = p.rb;
            g_sm.pre[k] = p.re;
            if (k == M_LM) off = 0;  // the LM head follows the last layer
            g_sm.poff[k] = off;
            off += (p.re - p.rb) * (p.K / CHUNK);
            if (k == M_DOWN) g_sm.ulayer = off;
        }
        for (int w = 0; w < NLOAD; ++w) g_sm.landed[w] = 0;
        for (int c = 0; c < NCOMP; ++c) g_sm.prog[c] = 0;
        g_sm.ready = 0;
        g_sm.done = 0;
        g_sm.abort = 0;
    }
    __syncthreads();
    if (wave < NLOAD) loader(ka, wave, lane);
    else if (wave < CTL_WAVE) compute(ka, wave - NLOAD, lane);
    else control(ka, lane, blockIdx.x, gridDim.x);
}

// Work buffer: [state 256 B][resid_x][qkv_x][attn_x][act_x][part_x][lm_x], 256-byte aligned pieces.
struct WorkLayout {
    size_t resid, qkv, attn, act, part, lm, total;
};
__host__ __device__ inline size_t align256(size_t v) { return (v + 255) & ~(size_t)255; }
inline WorkLayout work_layout(int H, int I, int Hq, int Hkv, int grid) {
    WorkLayout w;
    size_t off = 256;
    w.resid = off; off = align256(off + (size_t)H * 4);
    w.qkv = off; off = align256(off + (size_t)(Hq + 2 * Hkv) * PD * 4);
    w.attn = off; off = align256(off + (size_t)Hq * PD * 4);
    w.act = off; off = align256(off + (size_t)I * 4);
    w.part = off; off = align256(off + (size_t)grid * PGROUP * PREC * 4);  // Hkv * (grid / Hkv) ranges
    w.lm = off; off = align256(off + (size_t)grid * 16);
    w.total = off;
    return w;
}

int check_shapes(int L, int H, int I, int V, int Hq, int Hkv, int capacity, int grid) {
    if (L < 1 || capacity < 1 || V < 1 || Hkv < 1 || Hq != PGROUP * Hkv || grid < 1) return -1;
    if (H % CHUNK || H > 8 * CHUNK || I % CHUNK || I > MAX_X || (Hq * PD) % CHUNK || Hq * PD > MAX_X) return -1;
    if (grid % Hkv || grid / Hkv > MAX_SPLITS) return -1;
    const int T = Hq * PD;
    if (T % grid || T / grid > MAX_SLICE || PD % (T / grid)) return -1;
    const int qkv_rows = (Hq + 2 * Hkv) * PD;
    if ((qkv_rows + grid - 1) / grid > MAX_ROWS || 2 * ((I + grid - 1) / grid) > MAX_ROWS) return -1;
    if ((V + grid - 1) / grid > MAX_ROWS || (H + grid - 1) / grid > MAX_OWN) return -1;
    if ((H / grid) < 1) return -1;
    // 32-bit row partitions: n * grid must stay below 2^31 for every split matrix.
    const int64_t big = (int64_t)grid * (V > qkv_rows ? (V > I ? V : I) : (qkv_rows > I ? qkv_rows : I));
    if (big >= ((int64_t)1 << 31) || (int64_t)grid * Hq * PD >= ((int64_t)1 << 31)) return -1;
    return 0;
}

}  // namespace

extern "C" int q3_persist_grid(void) {
    // Workgroups that can be resident together on the current device: one per
    // CU (the LDS request admits no second).  0 if the kernel cannot run here.
    constexpr int MAX_DEV = 64;
    static int cached[MAX_DEV];  // 0 = not yet asked; -1 = cannot run; else the CU count
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess) return 0;
    if (dev >= 0 && dev < MAX_DEV && cached[dev] != 0) return cached[dev] > 0 ? cached[dev] : 0;
    int cus = 0, per_cu = 0;
    const bool ok =
        hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) == hipSuccess &&
        hipFuncSetAttribute(reinterpret_cast<const void*>(decode_persist_kernel),
                            hipFuncAttributeMaxDynamicSharedMemorySize, (int)(LDS_BYTES - sizeof(Smem))) == hipSuccess &&
        hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, decode_persist_kernel, PTHREADS, LDS_BYTES - sizeof(Smem)) ==
            hipSuccess &&
        per_cu >= 1 && cus > 0;
    if (dev >= 0 && dev < MAX_DEV) cached[dev] = ok ? cus : -1;
    return ok ? cus : 0;
}

extern "C" int q3_persist_supported(int L, int H, int I, int V, int Hq, int Hkv, int capacity, int grid) {
    return check_shapes(L, H, I, V, Hq, Hkv, capacity, grid) == 0 ? 1 : 0;
}

extern "C" int q3_persist_trace_words(int L, int grid) { return L < 1 || grid < 1 ? 0 : trace_words_all(L, grid); }

extern "C" int64_t q3_persist_work_bytes(int H, int I, int Hq, int Hkv, int grid) {
    return (int64_t)work_layout(H, I, Hq, Hkv, grid).total;
}

extern "C" int q3_decode_persistent(const q3_layer* layers, int L, const uint16_t* embed,
                                    const uint16_t* final_norm, const uint16_t* lm_head, int H, int I, int V,
                                    int Hq, int Hkv, const uint16_t* cos_t, const uint16_t* sin_t,
                                    uint16_t* cache_k, uint16_t* cache_v, int capacity, int64_t* tokens,
                                    int64_t* pos, void* work, int grid, uint16_t* logits, float eps, float scale,
                                    uint64_t* trace, hipStream_t stream) {
    if (!layers || !embed || !final_norm || !lm_head || !cos_t || !sin_t || !cache_k || !cache_v || !tokens ||
        !pos || !work)
        return (int)hipErrorInvalidValue;
    if (check_shapes(L, H, I, V, Hq, Hkv, capacity, grid) != 0) return (int)hipErrorInvalidValue;
    if ((reinterpret_cast<uintptr_t>(embed) | reinterpret_cast<uintptr_t>(lm_head) |
         reinterpret_cast<uintptr_t>(work)) & 255)
        return (int)hipErrorInvalidValue;
    // Every workgroup must be resident at once: one per CU.
    const int cus = q3_persist_grid();
    if (cus < 1 || grid > cus) return (int)hipErrorInvalidConfiguration;
    const WorkLayout w = work_layout(H, I, Hq, Hkv, grid);
    unsigned char* base = static_cast<unsigned char*>(work);
    PArgs a;
    a.layers = layers;
    a.embed = embed;
    a.final_norm = final_norm;
    a.lm_head = lm_head;
    a.cos_t = cos_t;
    a.sin_t = sin_t;
    a.cache_k = cache_k;
    a.cache_v = cache_v;
    a.tokens = tokens;
    a.pos = pos;
    a.logits = logits;
    a.state = reinterpret_cast<uint32_t*>(base);
    a.resid_x = reinterpret_cast<uint32_t*>(base + w.resid);
    a.qkv_x = reinterpret_cast<uint32_t*>(base + w.qkv);
    a.attn_x = reinterpret_cast<uint32_t*>(base + w.attn);
    a.act_x = reinterpret_cast<uint32_t*>(base + w.act);
    a.part_x = reinterpret_cast<uint32_t*>(base + w.part);
    a.lm_x = reinterpret_cast<uint32_t*>(base + w.lm);
    a.trace = trace;
    a.L = L; a.H = H; a.I = I; a.V = V; a.Hq = Hq; a.Hkv = Hkv; a.capacity = capacity;
    a.eps = eps;
    a.scale = scale;
    Q3_LAUNCH(decode_persist_kernel, dim3(grid), dim3(PTHREADS), LDS_BYTES - sizeof(Smem), stream, a);
    Q3_CHECK_LAUNCH();
}
