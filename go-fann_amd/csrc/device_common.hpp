// device_common.hpp -- device-side building blocks of the gfx950 search
// path: visited hash, symmetric min-max frontier heap, bounded binary heaps,
// CSR/DNF predicates, range atoms, early stop and wave64 reductions.
//
// Every routine keeps the observable semantics of the GO-FANN routine it
// cites (paths relative to the GO-FANN source tree); the layout and
// parallelisation are this file's own (wave64, LDS-resident state).
#pragma once

#include <hip/hip_runtime.h>

#include <cfloat>
#include <cstdint>

#include "gofann_hip.h"

namespace gofann {

// popcount(x) + acc as one v_bcnt_u32_b32.  Written out because the
// compiler otherwise counts each word on its own (bcnt x, 0) and sums the
// counts with extra adds -- a third more VALU work in the RaBitQ inner loops.
__device__ __forceinline__ uint32_t bcnt_acc(uint32_t x, uint32_t acc)
{
    uint32_t r;
    asm("v_bcnt_u32_b32 %0, %1, %2" : "=v"(r) : "v"(x), "v"(acc));
    return r;
}

// 16-byte code vectors a per-lane RaBitQ scorer loads before using any.
#ifndef GOFANN_CODE_BATCH
#define GOFANN_CODE_BATCH 8
#endif
constexpr int kCodeBatch = GOFANN_CODE_BATCH;

// Sum of x over the G-lane group holding this lane (G a power of two <= 32),
// delivered to every lane of the group; every lane of the group is active.
template <int G>
__device__ __forceinline__ int group_sum(int x)
{
    if constexpr (G >= 2) x += __builtin_amdgcn_mov_dpp(x, 0xB1, 0xF, 0xF, false);   // lane ^ 1
    if constexpr (G >= 4) x += __builtin_amdgcn_mov_dpp(x, 0x4E, 0xF, 0xF, false);   // lane ^ 2
    if constexpr (G >= 8) x += __builtin_amdgcn_mov_dpp(x, 0x141, 0xF, 0xF, false);  // 7 - lane in 8
    if constexpr (G >= 16) x += __builtin_amdgcn_mov_dpp(x, 0x140, 0xF, 0xF, false); // 15 - lane in 16
    if constexpr (G >= 32) x += __shfl_xor(x, 16, 64);
    return x;
}

// Wave-uniform minimum of x: DPP inside each 16-lane row, then the four
// row minima.
__device__ __forceinline__ uint32_t wave_min_u32(uint32_t x)
{
    x = min(x, static_cast<uint32_t>(__builtin_amdgcn_mov_dpp(static_cast<int>(x), 0xB1, 0xF, 0xF, false)));
    x = min(x, static_cast<uint32_t>(__builtin_amdgcn_mov_dpp(static_cast<int>(x), 0x4E, 0xF, 0xF, false)));
    x = min(x, static_cast<uint32_t>(__builtin_amdgcn_mov_dpp(static_cast<int>(x), 0x141, 0xF, 0xF, false)));
    x = min(x, static_cast<uint32_t>(__builtin_amdgcn_mov_dpp(static_cast<int>(x), 0x140, 0xF, 0xF, false)));
    const uint32_t a = static_cast<uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(x), 0));
    const uint32_t b = static_cast<uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(x), 16));
    const uint32_t c = static_cast<uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(x), 32));
    const uint32_t d = static_cast<uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(x), 48));
    return min(min(a, b), min(c, d));
}



constexpr uint32_t kHashCapacity = 4096;  // backend_pq.cu:194
constexpr int kMaxDegree = 64;            // include/config1B.h:29 FIXED_DEGREE
constexpr uint32_t kPoolUsed = 0x80000000u;  // backend_pq.cu:713
constexpr int kMaxStopWidth = 10;         // backend_pq.cu:72 kTopk
constexpr int kWave = 64;

// Frontier entry: priority `first`, label-local row | used bit, unbiased
// score `base` (gpu_predicate::BiasedPair, gpu_predicate_index.cuh:137-144)
// and the row's sample id, carried so that expanding the entry needs no
// row -> sample lookup (16 B, one ds_read_b128).
struct alignas(16) Entry {  // one 16-byte LDS access per entry
    float first;
    uint32_t second;
    float base;
    uint32_t sample;
};

struct ResultEntry {  // KernelPair<dist_t, uint32_t>
    float first;
    uint32_t second;
};

struct StopEntry {  // KernelPair<dist_t, idx_t>
    float first;
    uint32_t pad;
    uint64_t second;
};

__device__ __forceinline__ uint32_t fbits(float f) { return __float_as_uint(f); }
__device__ __forceinline__ float bitsf(uint32_t u) { return __uint_as_float(u); }

__device__ __forceinline__ int lane_id() { return static_cast<int>(threadIdx.x) & (kWave - 1); }

// Wave-uniform broadcast of lane 0's value.
__device__ __forceinline__ int bcast0(int v) { return __builtin_amdgcn_readlane(v, 0); }
__device__ __forceinline__ uint32_t bcast0u(uint32_t v)
{
    return static_cast<uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(v), 0));
}
__device__ __forceinline__ float bcast0f(float v)
{
    return bitsf(static_cast<uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(fbits(v)), 0)));
}

__device__ __forceinline__ uint64_t ballot(bool p) { return __ballot(p); }

// Number of set bits of `mask` below this lane (exclusive prefix).
__device__ __forceinline__ uint32_t lanes_below(uint64_t mask)
{
    return __builtin_amdgcn_mbcnt_hi(static_cast<uint32_t>(mask >> 32),
                                     __builtin_amdgcn_mbcnt_lo(static_cast<uint32_t>(mask), 0u));
}

// The lane id behind an empty asm statement.  A route loop that takes its
// lane from here at the top of every step recomputes what it derives from
// the lane (lane masks such as (1 << lane) - 1, per-lane addresses) where it
// is used, instead of the compiler hoisting those values out of the loop and
// holding them, or spilling them, for the whole route.
__device__ __forceinline__ int opaque_lane(int lane)
{
    asm volatile("" : "+v"(lane));
    return lane;
}

// ---------------------------------------------------------------------------
// Visited set: native_visited_hash.cuh:10-60.  Observable semantics: an exact
// set of label-local rows that stops accepting values once it holds 4096 of
// them (add drops silently when the 4096-slot table is full; test answers
// membership).  Any exact set with that capacity rule is indistinguishable,
// so the storage is chosen for residency:
//   kVisitedLds    the 4096-slot linear-probing table in LDS (16 KiB);
//   kVisitedGlobal the same table in a per-route global slab (agent-scope
//                  atomics, so lanes see each other's inserts past L1);
//   kVisitedSpill  a 1024-slot LDS table (4 KiB) that moves into the global
//                  table before its load passes 3/4 -- long routes only.
// Inserts of one step run lane-parallel (compare-and-swap) while the set
// cannot fill; otherwise lane 0 adds in admission order, reproducing which
// values the reference drops.
// ---------------------------------------------------------------------------
__device__ __forceinline__ uint32_t hash_code(uint32_t value)
{
    const uint64_t mixed = static_cast<uint64_t>(value) ^
                           (static_cast<uint64_t>(value >> 16) * 0x4bcb391f924ed183ULL) ^
                           0xa0ab69ccd854fc0aULL;
    return static_cast<uint32_t>(mixed % kHashCapacity);
}

constexpr int kVisitedGlobal = 0;
constexpr int kVisitedLds = 1;
constexpr int kVisitedSpill = 2;
constexpr uint32_t kSpillSlots = 1024;
constexpr uint32_t kSpillLimit = kSpillSlots * 3 / 4;

// Linear-probing table over `cap` slots (a power of two dividing 4096).
template <bool kShared>
struct ProbeTable {
    uint32_t* slots;
    uint32_t cap;

    __device__ __forceinline__ uint32_t load(uint32_t i) const
    {
        if constexpr (kShared) return slots[i];
        return __hip_atomic_load(slots + i, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    __device__ __forceinline__ void store(uint32_t i, uint32_t v) const
    {
        if constexpr (kShared) {
            slots[i] = v;
        } else {
            __hip_atomic_store(slots + i, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
    }
    __device__ void clear(int lane) const
    {
        uint4* p = reinterpret_cast<uint4*>(slots);
        const uint4 empty = make_uint4(UINT32_MAX, UINT32_MAX, UINT32_MAX, UINT32_MAX);
        for (uint32_t i = lane; i < cap / 4; i += kWave) p[i] = empty;
    }
    __device__ bool test(uint32_t value) const
    {
        uint32_t slot = hash_code(value) & (cap - 1);
        for (uint32_t probes = 0; probes < cap; ++probes) {
            const uint32_t v = load(slot);
            if (v == UINT32_MAX) return false;
            if (v == value) return true;
            slot = (slot + 1) & (cap - 1);
        }
        return false;
    }
    // Serial insert: 1 when stored, 0 when present or the table is full.
    __device__ int add(uint32_t value) const
    {
        uint32_t slot = hash_code(value) & (cap - 1);
        for (uint32_t probes = 0; probes < cap; ++probes) {
            const uint32_t v = load(slot);
            if (v == value) return 0;
            if (v == UINT32_MAX) {
                store(slot, value);
                return 1;
            }
            slot = (slot + 1) & (cap - 1);
        }
        return 0;
    }
    // Lane-parallel insert; the caller guarantees a free slot for every
    // inserting lane.  1 when this lane stored the value.
    __device__ int add_parallel(uint32_t value) const
    {
        uint32_t slot = hash_code(value) & (cap - 1);
        for (uint32_t probes = 0; probes < cap; ++probes) {
            uint32_t expected = UINT32_MAX;
            if constexpr (kShared) {
                expected = atomicCAS(slots + slot, UINT32_MAX, value);
            } else {
                __hip_atomic_compare_exchange_strong(slots + slot, &expected, value,
                                                     __ATOMIC_RELAXED, __ATOMIC_RELAXED,
                                                     __HIP_MEMORY_SCOPE_AGENT);
            }
            if (expected == UINT32_MAX) return 1;
            if (expected == value) return 0;
            slot = (slot + 1) & (cap - 1);
        }
        return 0;
    }
};

template <int kMode>
struct VisitedSet {
    ProbeTable<true> shared;    // LDS table (kVisitedLds, kVisitedSpill)
    ProbeTable<false> global;   // global slab of 4096 slots
    uint32_t count;             // values held (wave-uniform)
    bool spilled;               // kVisitedSpill: moved to the global slab

    __device__ void init(uint32_t* lds_slots, uint32_t* global_slots, int lane)
    {
        shared = {lds_slots, kMode == kVisitedSpill ? kSpillSlots : kHashCapacity};
        global = {global_slots, kHashCapacity};
        count = 0;
        spilled = false;
        if constexpr (kMode == kVisitedGlobal) {
            global.clear(lane);
        } else {
            shared.clear(lane);
        }
    }
    __device__ __forceinline__ bool in_global() const
    {
        return kMode == kVisitedGlobal || (kMode == kVisitedSpill && spilled);
    }
    __device__ bool test(uint32_t value) const
    {
        return in_global() ? global.test(value) : shared.test(value);
    }
    // Lane 0 only; the caller broadcasts the result into `count`.  A full
    // set ignores adds (the probe would find neither the value's slot nor
    // an empty one), so `added` tracks the values stored by this batch.
    __device__ int add_serial(uint32_t value, uint32_t added) const
    {
        if (count + added >= kHashCapacity) return 0;
        return in_global() ? global.add(value) : shared.add(value);
    }
    __device__ int add_parallel(uint32_t value) const
    {
        return in_global() ? global.add_parallel(value) : shared.add_parallel(value);
    }
    // All lanes, before inserting `incoming` more values: move the small LDS
    // table into the global slab when it would pass its load limit.
    __device__ void reserve(uint32_t incoming, int lane)
    {
        if constexpr (kMode == kVisitedSpill) {
            if (spilled || count + incoming <= kSpillLimit) return;
            global.clear(lane);
            __threadfence();
            __syncthreads();
            for (uint32_t i = lane; i < kSpillSlots; i += kWave) {
                const uint32_t v = shared.slots[i];
                if (v != UINT32_MAX) (void)global.add_parallel(v);
            }
            __threadfence();
            __syncthreads();
            spilled = true;
        }
    }
};

// ---------------------------------------------------------------------------
// Symmetric min-max heap (include/smmh2.h:1-147): slot 0 empty, slot 1 =
// minimum, slot 2 = maximum; comparisons on `first` only.  Executed by one
// lane; the array lives in LDS.
// ---------------------------------------------------------------------------
__device__ __forceinline__ void entry_swap(Entry* a, Entry* b)
{
    const Entry t = *a;
    *a = *b;
    *b = t;
}

__device__ __forceinline__ int smmh_adjust_sibling(Entry* h, int y, int size)
{
    if (y & 1) {
        const int s = y + 1;
        if (s >= size) return y;
        if (h[y].first > h[s].first) {
            entry_swap(&h[y], &h[s]);
            return s;
        }
    } else {
        const int s = y - 1;
        if (h[y].first < h[s].first) {
            entry_swap(&h[y], &h[s]);
            return s;
        }
    }
    return y;
}

__device__ __forceinline__ int smmh_adjust_grandparent(Entry* h, int y)
{
    if (y <= 2) return y;
    const int g = (y - 3) >> 2;
    const int gl = (g << 1) + 1;
    const int gr = (g << 1) + 2;
    if (h[gl].first > h[y].first) {
        entry_swap(&h[gl], &h[y]);
        return gl;
    } else if (h[gr].first < h[y].first) {
        entry_swap(&h[gr], &h[y]);
        return gr;
    }
    return y;
}

__device__ __forceinline__ void smmh_insert(Entry* h, int& size, const Entry& e)
{
    int y = size;
    h[size++] = e;
    for (;;) {
        y = smmh_adjust_sibling(h, y, size);
        const int x = smmh_adjust_grandparent(h, y);
        if (x == y) break;
        y = x;
    }
}

__device__ __forceinline__ int smmh_adjust_grandchild(Entry* h, int y, int size)
{
    if (y & 1) {
        const int cl = (y << 1) + 1;
        if (cl >= size) return y;
        const int cr = ((y + 1) << 1) + 1;
        int c = cl;
        if (cr < size && h[cr].first < h[cl].first) c = cr;
        if (h[c].first < h[y].first) {
            entry_swap(&h[c], &h[y]);
            return c;
        }
    } else {
        const int cl = ((y - 1) << 1) + 2;
        const int cr = (y << 1) + 2;
        if (cl >= size) return y;
        int c = cl;
        if (cr < size && h[cr].first > h[cl].first) c = cr;
        if (h[c].first > h[y].first) {
            entry_swap(&h[c], &h[y]);
            return c;
        }
    }
    return y;
}

__device__ __forceinline__ void smmh_pop_max(Entry* h, int& size)
{
    h[2] = h[--size];
    int y = 2;
    for (;;) {
        (void)smmh_adjust_sibling(h, y, size);
        const int x = smmh_adjust_grandchild(h, y, size);
        if (x == y) break;
        y = x;
    }
}

// ---------------------------------------------------------------------------
// The same two operations executed by the whole wave, for a heap of at most
// 512 slots (256 pairs), leaving the array exactly as smmh_insert /
// smmh_pop_max do (tie for tie); every lane passes the same arguments.
//
// Insert: after the bottom sibling step the new entry only ever moves up
// one chain -- the left slots of its ancestor pairs when it is below the
// parent pair's minimum, the right slots when it is above the maximum --
// and the sifted values along a chain are sorted, so the levels it climbs
// are a prefix of that chain.  Lane j reads both slots of ancestor j (and
// every lane the new slot's sibling) in one round trip, a ballot counts
// the prefix, the prefix moves down one level and the entry lands on top.
//
// Pop max: the serial sift walks from slot 2 to the larger right slot of
// the two child pairs at every level; that walk depends only on values
// below it, so lane q compares pair q's two children (and pair q + 64's in
// a heap over 260 slots), a ballot packs the picks, and the walk is a
// scalar loop over those bits.  Lane k then holds path slot k and its left
// sibling.  The moving value after level k is the maximum of itself and
// the left siblings of levels 0..k (a swap takes a strictly larger left
// entry), a prefix maximum over the path lanes; it stops at the first level
// whose next path slot is not larger.  The writes are parallel.
// ---------------------------------------------------------------------------
__device__ __forceinline__ Entry shfl_entry(const Entry& e, int src)
{
    Entry r;
    r.first = __int_as_float(__shfl(__float_as_int(e.first), src, kWave));
    r.second = static_cast<uint32_t>(__shfl(static_cast<int>(e.second), src, kWave));
    r.base = __int_as_float(__shfl(__float_as_int(e.base), src, kWave));
    r.sample = static_cast<uint32_t>(__shfl(static_cast<int>(e.sample), src, kWave));
    return r;
}

__device__ __forceinline__ Entry readlane_entry(const Entry& e, int src)
{
    Entry r;
    r.first = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(e.first), src));
    r.second = static_cast<uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(e.second), src));
    r.base = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(e.base), src));
    r.sample = static_cast<uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(e.sample), src));
    return r;
}

// DPP moves within rows of 16 lanes; a lane whose source is outside its row
// keeps `old`.  Row shift right by n: lane i reads lane i - n; row shift
// left by 1: lane i reads lane i + 1.
template <int kCtrl>
__device__ __forceinline__ int dpp_row(int old, int x)
{
    return __builtin_amdgcn_update_dpp(old, x, kCtrl, 0xF, 0xF, false);
}
template <int kCtrl>
__device__ __forceinline__ float dpp_row_f(float old, float x)
{
    return __int_as_float(dpp_row<kCtrl>(__float_as_int(old), __float_as_int(x)));
}
constexpr int kDppRowShl1 = 0x101;
constexpr int kDppRowShr1 = 0x111;
constexpr int kDppRowShr2 = 0x112;
constexpr int kDppRowShr4 = 0x114;
constexpr int kDppRowShr8 = 0x118;

constexpr int kWaveHeapSlots = 512;  // slots 0..511: 256 pairs, paths of <= 8 levels

__device__ __forceinline__ Entry select_entry(bool c, const Entry& a, const Entry& b)
{
    Entry r;
    r.first = c ? a.first : b.first;
    r.second = c ? a.second : b.second;
    r.base = c ? a.base : b.base;
    r.sample = c ? a.sample : b.sample;
    return r;
}

__device__ __forceinline__ void wave_smmh_insert(Entry* h, int& size, const Entry& e, int lane)
{
    const int y0 = __builtin_amdgcn_readfirstlane(size);
    size = y0 + 1;
    // the pair of slot y0 (and of y0 - 1 when y0 is even); its ancestor pairs
    const int pair = (y0 - 1) >> 1;
    const int depth = pair > 0 ? 31 - __clz(pair + 1) : 0;
    const bool act = lane >= 1 && lane <= depth;
    // lanes past the chain read slots 1 and 2 (inside the frontier) and stay out
    const int a1 = act ? 2 * (((pair + 1) >> lane) - 1) + 1 : 1;
    const Entry al = h[a1];
    const Entry ar = h[a1 + 1];
    const Entry sib = h[y0 - 1];
    // bottom sibling step: the pair's left entry moves right (lane 63 writes it)
    const bool moved =
        !(y0 & 1) && e.first < __int_as_float(__builtin_amdgcn_readfirstlane(__float_as_int(sib.first)));
    const int y = moved ? y0 - 1 : y0;
    // side 0 climbs the left (minimum) slots, 1 the right slots, -1 stays
    int side = -1;
    if (depth > 0) {
        if (__int_as_float(__builtin_amdgcn_readlane(__float_as_int(al.first), 1)) > e.first)
            side = 0;
        else if (__int_as_float(__builtin_amdgcn_readlane(__float_as_int(ar.first), 1)) < e.first)
            side = 1;
    }
    const Entry v = select_entry(side == 1, ar, al);
    const float sg = side == 1 ? -1.0f : 1.0f;  // climb: v > e on the left side, v < e on the right
    const uint64_t mask = ballot(side >= 0 && act && sg * v.first > sg * e.first);
    const int t = __builtin_ctzll(~(mask >> 1));  // levels climbed (0 when it stays)
    const int sd = side == 1 ? 1 : 0;
    // lane 0: the new entry; lanes 1..t: the chain moves down one level
    const int lv = lane == 0 ? t : lane - 1;
    int dst = lv == 0 ? y : 2 * (((pair + 1) >> lv) - 1) + 1 + sd;
    Entry w = select_entry(lane == 0, e, v);
    bool wr = lane == 0 || (act && lane <= t);
    if (lane == kWave - 1) {
        dst = y0;
        w = sib;
        wr = moved;
    }
    if (wr) h[dst] = w;
}

// Returns the new maximum (slot 2's `first`); the heap keeps >= 3 slots.
__device__ __forceinline__ float wave_smmh_pop_max(Entry* h, int& size, int lane)
{
    const int n = __builtin_amdgcn_readfirstlane(size) - 1;
    size = n;
    const Entry v = h[n];  // the last entry replaces the maximum
    // bit q: pair q's larger child is its right one (ties: the left)
    uint64_t pick0, pick1 = 0;
    {
        const int cl = 4 * lane + 4;
        const int cr = cl + 2;
        const float fl = h[min(cl, n - 1)].first;
        const float fr = h[min(cr, n - 1)].first;
        pick0 = ballot(cr < n && fr > fl);
        if (n > 260) {
            const float gl = h[min(cl + 256, n - 1)].first;
            const float gr = h[min(cr + 256, n - 1)].first;
            pick1 = ballot(cr + 256 < n && gr > gl);
        }
    }
    int p = 0;  // scalar walk to the last pair of the path
    int depth = 0;
    while (4 * p + 4 < n) {
        const uint64_t bits = p < kWave ? pick0 : pick1;
        p = 2 * p + 1 + static_cast<int>((bits >> (p & (kWave - 1))) & 1ull);
        ++depth;
    }
    // lane k <= depth: path slot k; lanes past the path read slot 2
    const int k = lane <= depth ? lane : 0;
    const int slot = 2 * (((p + 1) >> (depth - k)) - 1) + 2;
    const Entry R = h[slot];
    const Entry L = h[slot - 1];
    float x = L.first;
    const float ninf = -__builtin_inff();
    x = fmaxf(x, dpp_row_f<kDppRowShr1>(ninf, x));
    x = fmaxf(x, dpp_row_f<kDppRowShr2>(ninf, x));
    x = fmaxf(x, dpp_row_f<kDppRowShr4>(ninf, x));
    x = fmaxf(x, dpp_row_f<kDppRowShr8>(ninf, x));
    const float vf = fmaxf(v.first, x);                        // after level `lane`
    const float prev = dpp_row_f<kDppRowShr1>(v.first, vf);    // entering level `lane`
    const uint64_t swapped = ballot(lane <= depth && L.first > prev);
    Entry rnext;  // path slot lane + 1
    rnext.first = dpp_row_f<kDppRowShl1>(R.first, R.first);
    rnext.second = static_cast<uint32_t>(dpp_row<kDppRowShl1>(static_cast<int>(R.second), static_cast<int>(R.second)));
    rnext.base = dpp_row_f<kDppRowShl1>(R.base, R.base);
    rnext.sample = static_cast<uint32_t>(dpp_row<kDppRowShl1>(static_cast<int>(R.sample), static_cast<int>(R.sample)));
    const int stop = __builtin_ctzll(~ballot(lane < depth && rnext.first > vf));
    // entering level k: the last left entry swapped in above k, else v
    const uint64_t above = swapped & ((1ull << lane) - 1ull);
    const Entry lsrc = shfl_entry(L, above ? 63 - __builtin_clzll(above) : 0);
    // where it stops: the left entry swapped in there or above, else v
    const uint64_t upto = swapped & ((2ull << stop) - 1ull);
    const Entry lfin = readlane_entry(L, upto ? 63 - __builtin_clzll(upto) : 0);
    const Entry fin = select_entry(upto != 0, lfin, v);
    if (lane <= stop) {
        h[slot] = select_entry(lane == stop, fin, rnext);
        if ((swapped >> lane) & 1ull) h[slot - 1] = select_entry(above != 0, lsrc, v);
    }
    return stop == 0 ? fin.first : __int_as_float(__builtin_amdgcn_readlane(__float_as_int(R.first), 1));
}

// ---------------------------------------------------------------------------
// Bounded max-heaps of include/bin_heap.h:4-64 (push sifts the appended
// element up; pop returns the root and sifts the former tail down without
// storing the root at the tail).
// ---------------------------------------------------------------------------
template <class T>
__device__ __forceinline__ void bin_push(T* h, int size)
{
    int now = size - 1;
    int parent = (now - 1) / 2;
    while (now > 0 && h[parent].first < h[now].first) {
        const T t = h[now];
        h[now] = h[parent];
        h[parent] = t;
        now = parent;
        parent = (now - 1) / 2;
    }
}

template <class T>
__device__ __forceinline__ T bin_pop(T* h, int size)
{
    const T ret = h[0];
    const int len = size - 1;
    if (len <= 0) return ret;
    h[0] = h[size - 1];
    int now = 0;
    while (now * 2 + 1 < len) {
        const int left = now * 2 + 1;
        const int right = now * 2 + 2;
        int next = left;
        if (right < len && h[left].first < h[right].first) next = right;
        if (!(h[now].first < h[next].first)) break;
        const T t = h[now];
        h[now] = h[next];
        h[next] = t;
        now = next;
    }
    return ret;
}

// ---------------------------------------------------------------------------
// Posting shortlist order (posting_shortlist_heap.cuh:15-21): a pair is worse
// when its distance is larger, ties broken by the larger id.
// ---------------------------------------------------------------------------
__device__ __forceinline__ bool pair_worse(float ld, uint32_t lid, float rd, uint32_t rid)
{
    return ld > rd || (ld == rd && lid > rid);
}

// ---------------------------------------------------------------------------
// Early stop: backend_pq.cu:2822-2873.
// ---------------------------------------------------------------------------
__device__ __forceinline__ int adaptive_limit(int queue_limit, int expanded, int passed,
                                              int stop_width)
{
    const int queue_base = queue_limit > 1 ? queue_limit : 1;
    int base_limit = (queue_base + 1) / 2;
    const int min_base = stop_width > 0 ? stop_width * 2 : 1;
    base_limit = base_limit > min_base ? base_limit : min_base;
    const int denom = (expanded + 16) > 1 ? (expanded + 16) : 1;
    const int pass_with_prior = passed + 8;
    const int pass_estimate = pass_with_prior < denom ? pass_with_prior : denom;
    const int reject_estimate = (denom - pass_estimate) > 0 ? (denom - pass_estimate) : 0;
    const int64_t numerator = static_cast<int64_t>(queue_limit) * reject_estimate;
    int extra = static_cast<int>((numerator + (2 * denom - 1)) / (2 * denom));
    extra = extra > 0 ? extra : 0;
    extra = extra < 32 ? extra : 32;
    return base_limit + extra;
}

__device__ __forceinline__ bool early_stop_reached(int mode, int bad, int fixed_limit,
                                                   int queue_limit, int expanded, int passed,
                                                   int stop_width)
{
    if (mode == GOFANN_EARLY_STOP_OFF) return false;
    if (mode == GOFANN_EARLY_STOP_ADAPTIVE)
        return bad >= adaptive_limit(queue_limit, expanded, passed, stop_width);
    return bad >= fixed_limit;
}

// ---------------------------------------------------------------------------
// Predicates: gpu_predicate_index.cuh:52-166 (CSR storage, threshold 0) and
// range_filter.cuh:23-124.
// ---------------------------------------------------------------------------
// Attribute columns of a predicate view's base_ranges.
__device__ __forceinline__ uint32_t range_columns(const gofann_predicate_view& v)
{
    return v.range_columns ? v.range_columns : v.range_stride;
}

struct PredCounters {
    uint32_t rows;
    uint32_t labels;
};

__device__ __forceinline__ bool range_matches(uint32_t mode, float lower, float upper, float v)
{
    switch (mode) {
    case 0: return true;
    case 1: return v > lower;
    case 2: return v < upper;
    case 3: return v >= lower && v < upper;
    default: return false;
    }
}

__device__ __forceinline__ bool pred_enabled(const gofann_predicate_view& v, uint32_t route)
{
    return v.route_enabled ? v.route_enabled[route] != 0 : (v.csr_offsets != nullptr);
}

__device__ __forceinline__ bool pred_contains(const gofann_predicate_view& v, uint32_t handle,
                                              uint32_t sample, PredCounters& c)
{
    if (sample >= v.rows || v.csr_offsets == nullptr) return false;
    const uint32_t begin = v.csr_offsets[sample];
    const uint32_t end = v.csr_offsets[sample + 1];
    ++c.rows;
    for (uint32_t i = begin; i < end; ++i) {
        const uint32_t label = v.csr_labels[i];
        ++c.labels;
        if (label >= handle) return label == handle;
    }
    return false;
}

__device__ __forceinline__ bool pred_matches(const gofann_predicate_view& v, uint32_t route, uint32_t sample,
                             PredCounters& c)
{
    if (sample >= v.rows) return false;
    if (v.clauses) {
        for (uint32_t i = v.route_offsets[route]; i < v.route_offsets[route + 1]; ++i) {
            const gofann_clause cl = v.clauses[i];
            bool pass = true;
            for (uint32_t j = cl.label_begin; pass && j < cl.label_end; ++j)
                pass = pred_contains(v, v.route_handles[j], sample, c);
            for (uint32_t j = cl.range_begin; pass && j < cl.range_end; ++j) {
                const gofann_range_atom a = v.ranges[j];
                pass = v.base_ranges != nullptr && a.dimension < range_columns(v) &&
                       range_matches(a.mode, a.lower, a.upper,
                                     v.base_ranges[static_cast<uint64_t>(sample) * v.range_stride +
                                                   a.dimension]);
            }
            if (pass) return true;
        }
        return false;
    }
    for (uint32_t i = v.route_offsets[route]; i < v.route_offsets[route + 1]; ++i)
        if (!pred_contains(v, v.route_handles[i], sample, c)) return false;
    return true;
}

// Inline label slab (gofann_predicate_view.label_slab): 16 bytes per sample,
// u16 count then up to 7 u16 labels; count 0xFFFF = read the CSR row.
constexpr uint32_t kSlabCapacity = 7;
constexpr uint32_t kSlabOverflow = 0xFFFFu;

__device__ __forceinline__ bool slab_usable(const gofann_predicate_view& v, uint32_t sample)
{
    return v.label_slab != nullptr && v.csr_offsets != nullptr && sample < v.rows;
}

__device__ __forceinline__ uint4 slab_load(const gofann_predicate_view& v, uint32_t sample)
{
    return *reinterpret_cast<const uint4*>(v.label_slab + static_cast<size_t>(sample) * v.slab_stride);
}

__device__ __forceinline__ uint32_t slab_count(const uint4& w) { return w.x & 0xFFFFu; }

// Label k (0-based) of a slab; k may be a runtime value.
__device__ __forceinline__ uint32_t slab_label(const uint4& w, uint32_t k)
{
    const uint32_t h = k + 1;  // u16 index
    const uint32_t word = (h >> 1) == 0 ? w.x : (h >> 1) == 1 ? w.y : (h >> 1) == 2 ? w.z : w.w;
    return (word >> (16 * (h & 1))) & 0xFFFFu;
}

// One sample's CSR label row held across the wave: lane k holds label
// begin+k of the first 64 (UINT32_MAX past the end).  Loaded once per
// expanded node; every handle test of the route's clauses reads it.
struct WaveRow {
    uint32_t begin, end;  // wave-uniform bounds
    uint32_t lab;         // this lane's label of the first chunk
    bool valid;           // sample < rows and CSR present
};

__device__ __forceinline__ WaveRow wave_row_load(const gofann_predicate_view& v, uint32_t sample,
                                                 uint32_t begin, uint32_t end, int lane)
{
    WaveRow r;
    r.valid = sample < v.rows && v.csr_offsets != nullptr;
    r.begin = begin;
    r.end = r.valid ? end : begin;
    const uint32_t len = r.end - r.begin;
    r.lab = static_cast<uint32_t>(lane) < len ? v.csr_labels[r.begin + lane] : UINT32_MAX;
    return r;
}

// Wave-uniform csr_contains_sorted (gpu_predicate_index.cuh:58-78) over a
// WaveRow: the first label >= handle decides, and the number of labels the
// serial scan would have read is counted exactly.
__device__ __forceinline__ bool wave_row_contains(const gofann_predicate_view& v, const WaveRow& r,
                                  uint32_t handle, int lane, PredCounters& c)
{
    if (!r.valid) return false;
    ++c.rows;
    const uint32_t len = r.end - r.begin;
    for (uint32_t base = 0; base < len; base += kWave) {
        const uint32_t k = base + static_cast<uint32_t>(lane);
        const uint32_t lab = base == 0 ? r.lab : (k < len ? v.csr_labels[r.begin + k] : UINT32_MAX);
        const uint64_t ge = ballot(k < len && lab >= handle);
        if (ge) {
            const int f = __builtin_ctzll(ge);
            c.labels += base + static_cast<uint32_t>(f) + 1u;
            return static_cast<uint32_t>(__shfl(static_cast<int>(lab), f, kWave)) == handle;
        }
    }
    c.labels += len;
    return false;
}

// WaveRow of a sample whose inline slab (count != overflow) is at hand.
__device__ __forceinline__ WaveRow wave_row_from_slab(const uint4& slab, int lane)
{
    WaveRow r;
    r.valid = true;
    r.begin = 0;
    r.end = slab_count(slab);
    const uint32_t l = static_cast<uint32_t>(lane);
    r.lab = l < r.end && l < kSlabCapacity ? slab_label(slab, l) : UINT32_MAX;
    return r;
}

// pred_matches for a wave-uniform sample whose row is held in a WaveRow.
__device__ __forceinline__ bool wave_pred_matches(const gofann_predicate_view& v, uint32_t route, uint32_t sample,
                                  const WaveRow& row, int lane, PredCounters& c)
{
    if (sample >= v.rows) return false;
    if (v.clauses) {
        for (uint32_t i = v.route_offsets[route]; i < v.route_offsets[route + 1]; ++i) {
            const gofann_clause cl = v.clauses[i];
            bool pass = true;
            for (uint32_t j = cl.label_begin; pass && j < cl.label_end; ++j)
                pass = wave_row_contains(v, row, v.route_handles[j], lane, c);
            for (uint32_t j = cl.range_begin; pass && j < cl.range_end; ++j) {
                const gofann_range_atom a = v.ranges[j];
                pass = v.base_ranges != nullptr && a.dimension < range_columns(v) &&
                       range_matches(a.mode, a.lower, a.upper,
                                     v.base_ranges[static_cast<uint64_t>(sample) * v.range_stride +
                                                   a.dimension]);
            }
            if (pass) return true;
        }
        return false;
    }
    for (uint32_t i = v.route_offsets[route]; i < v.route_offsets[route + 1]; ++i)
        if (!wave_row_contains(v, row, v.route_handles[i], lane, c)) return false;
    return true;
}

// Per-lane pred_matches with the row's first labels loaded up front (one
// round of independent loads instead of a dependent chain); the serial
// decision order and the counters are those of pred_contains.
constexpr int kLaneRowBatch = 8;

struct LaneRow {
    uint32_t begin, end;
    uint32_t lab[kLaneRowBatch];  // UINT32_MAX past the end; constant-indexed only
};

__device__ __forceinline__ bool lane_row_contains(const gofann_predicate_view& v, const LaneRow& r,
                                                  uint32_t handle, PredCounters& c)
{
    ++c.rows;
    const uint32_t len = r.end - r.begin;
    // First batch position whose label is >= handle (the serial scan stops
    // there), found with constant indices so the batch stays in registers.
    uint32_t hit = static_cast<uint32_t>(kLaneRowBatch);
    bool eq = false;
#pragma unroll
    for (int k = 0; k < kLaneRowBatch; ++k) {
        const bool stop = hit == static_cast<uint32_t>(kLaneRowBatch) &&
                          static_cast<uint32_t>(k) < len && r.lab[k] >= handle;
        if (stop) {
            hit = static_cast<uint32_t>(k);
            eq = r.lab[k] == handle;
        }
    }
    if (hit < static_cast<uint32_t>(kLaneRowBatch)) {
        c.labels += hit + 1u;
        return eq;
    }
    if (len <= static_cast<uint32_t>(kLaneRowBatch)) {
        c.labels += len;
        return false;
    }
    c.labels += static_cast<uint32_t>(kLaneRowBatch);
    for (uint32_t i = r.begin + kLaneRowBatch; i < r.end; ++i) {
        const uint32_t label = v.csr_labels[i];
        ++c.labels;
        if (label >= handle) return label == handle;
    }
    return false;
}

// Three phases so a caller can overlap the row loads with other memory
// rounds: bounds (the slab, or CSR offsets), fill (the first labels), eval
// (clauses).  `slab` carries the slab words from bounds to fill.
__device__ __forceinline__ void lane_row_bounds(const gofann_predicate_view& v, uint32_t sample,
                                                bool active, LaneRow& r, uint4& slab)
{
    // computed in locals and stored once, so the row stays in registers
    uint32_t b = 0, e = 0;
    uint4 sl = make_uint4(kSlabOverflow, 0, 0, 0);
    const bool use_slab = active && slab_usable(v, sample);
    if (use_slab) {
        sl = slab_load(v, sample);
    } else if (active && sample < v.rows && v.csr_offsets != nullptr) {
        b = v.csr_offsets[sample];
        e = v.csr_offsets[sample + 1];
    }
    r.begin = b;
    r.end = e;
    slab = sl;
}

__device__ __forceinline__ void lane_row_fill(const gofann_predicate_view& v, LaneRow& r,
                                              uint32_t sample, const uint4& slab)
{
    if (slab_usable(v, sample)) {
        const uint32_t n = slab_count(slab);
        if (n != kSlabOverflow) {
            // The inline row: same labels, same scan, no memory access.
            r.begin = 0;
            r.end = n;
#pragma unroll
            for (int k = 0; k < kLaneRowBatch; ++k)
                r.lab[k] = static_cast<uint32_t>(k) < n && k < static_cast<int>(kSlabCapacity)
                               ? slab_label(slab, static_cast<uint32_t>(k))
                               : UINT32_MAX;
            return;
        }
    }
    // the bounds in locals (an overflowing slab reads them from the CSR), so
    // the row stays in registers
    const bool overflow = slab_usable(v, sample);
    const uint32_t b = overflow ? v.csr_offsets[sample] : r.begin;
    const uint32_t e = overflow ? v.csr_offsets[sample + 1] : r.end;
    r.begin = b;
    r.end = e;
    const uint32_t last = e > b ? e - 1 : b;
#pragma unroll
    for (int k = 0; k < kLaneRowBatch; ++k) {
        // Clamped address: every load is in bounds, so the batch issues as
        // independent loads; entries past the end are masked afterwards.
        const uint32_t i = b + static_cast<uint32_t>(k) < last ? b + k : last;
        const uint32_t x = e > b ? v.csr_labels[i] : UINT32_MAX;
        r.lab[k] = b + static_cast<uint32_t>(k) < e ? x : UINT32_MAX;
    }
}

__device__ __forceinline__ bool lane_pred_eval(const gofann_predicate_view& v, uint32_t route,
                                               uint32_t sample, const LaneRow& r, PredCounters& c)
{
    if (sample >= v.rows || v.csr_offsets == nullptr) return pred_matches(v, route, sample, c);
    if (v.clauses) {
        for (uint32_t i = v.route_offsets[route]; i < v.route_offsets[route + 1]; ++i) {
            const gofann_clause cl = v.clauses[i];
            bool pass = true;
            for (uint32_t j = cl.label_begin; pass && j < cl.label_end; ++j)
                pass = lane_row_contains(v, r, v.route_handles[j], c);
            for (uint32_t j = cl.range_begin; pass && j < cl.range_end; ++j) {
                const gofann_range_atom a = v.ranges[j];
                pass = v.base_ranges != nullptr && a.dimension < range_columns(v) &&
                       range_matches(a.mode, a.lower, a.upper,
                                     v.base_ranges[static_cast<uint64_t>(sample) * v.range_stride +
                                                   a.dimension]);
            }
            if (pass) return true;
        }
        return false;
    }
    for (uint32_t i = v.route_offsets[route]; i < v.route_offsets[route + 1]; ++i)
        if (!lane_row_contains(v, r, v.route_handles[i], c)) return false;
    return true;
}

__device__ __forceinline__ float priority(float base, float penalty, bool pass)
{
    if (pass || penalty == 0.0f || !isfinite(base) || base == FLT_MAX) return base;
    if (base > FLT_MAX - penalty) return FLT_MAX;
    return base + penalty;
}

__device__ __forceinline__ float bias_penalty(float alpha, float start)
{
    const double wide = static_cast<double>(alpha) * fmax(static_cast<double>(fabsf(start)), 1e-6);
    return isfinite(wide) ? static_cast<float>(fmin(wide, static_cast<double>(FLT_MAX))) : 0.0f;
}

__device__ __forceinline__ uint32_t count_active_ranges(const uint8_t* modes, uint32_t route,
                                                        uint32_t count)
{
    if (modes == nullptr) return 0;
    uint32_t active = 0;
    for (uint32_t r = 0; r < count; ++r)
        if (modes[static_cast<size_t>(route) * count + r] != 0) ++active;
    return active;
}

__device__ __forceinline__ uint32_t count_matching_ranges(const gofann_routes& rt, uint32_t route,
                                                          uint32_t sample)
{
    if (rt.range_modes == nullptr || rt.range_lower == nullptr || rt.range_upper == nullptr)
        return 0;
    uint32_t matched = 0;
    for (uint32_t r = 0; r < rt.range_count; ++r) {
        const size_t qf = static_cast<size_t>(route) * rt.range_count + r;
        const uint8_t mode = rt.range_modes[qf];
        if (mode == 0) continue;
        if (rt.base_range_values == nullptr) return 0;
        if (range_matches(mode, rt.range_lower[qf], rt.range_upper[qf],
                          rt.base_range_values[static_cast<size_t>(sample) * rt.range_count + r]))
            ++matched;
    }
    return matched;
}

__device__ __forceinline__ float apply_filter_bonuses(float dist, bool bit_match, uint32_t matched,
                                                      float bit_bonus, float range_bonus)
{
    if (bit_match) dist *= bit_bonus;
    for (uint32_t i = 0; i < matched; ++i) dist *= range_bonus;
    return dist;
}

// ---------------------------------------------------------------------------
// Wave64 reductions.
// ---------------------------------------------------------------------------
__device__ __forceinline__ float wave_min(float v)
{
    for (int off = 32; off > 0; off >>= 1) v = fminf(v, __shfl_xor(v, off, kWave));
    return v;
}

__device__ __forceinline__ int wave_sum(int v)
{
    for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off, kWave);
    return v;
}

// Float -> unsigned key of the same order (-0 folded onto +0, which compare
// equal as floats), and back.  Frontier keys are distances or priorities of
// finite vectors; a NaN would order above +inf.
__device__ __forceinline__ uint32_t order_key(float f)
{
    const uint32_t b = __float_as_uint(f == 0.0f ? 0.0f : f);
    return (b & 0x80000000u) ? ~b : (b | 0x80000000u);
}

__device__ __forceinline__ float order_key_float(uint32_t k)
{
    return __uint_as_float((k & 0x80000000u) ? (k & 0x7fffffffu) : ~k);
}

// Frontier pickup (wave-cooperative).
// pickup_next_unused_from_native_frontier (backend_pq.cu:844-892): unused
// entry of least `first`, lowest index on ties; lane 0 marks it used.
// Each lane scans slots lane + 1, lane + 65, ... in ascending order and
// keeps its first slot at its least key; then one unsigned wave minimum of
// the keys and one of the slots holding it (DPP row steps, no LDS
// permutes).  With `want_base`, the same pass also returns in `min_base`
// the least `base` over the entries that were unused before the pickup
// (the picked one included).
__device__ __forceinline__ bool pickup(Entry* f, int size, Entry& out, int lane,
                                       bool want_base, float& min_base)
{
    uint32_t bk = UINT32_MAX;
    uint32_t bi = UINT32_MAX;
    uint32_t mb = UINT32_MAX;
    for (int i = lane + 1; i < size; i += kWave) {
        const Entry e = f[i];
        if (e.second & kPoolUsed) continue;
        if (want_base) mb = min(mb, order_key(e.base));
        const uint32_t k = order_key(e.first);
        if (k < bk) {
            bk = k;
            bi = static_cast<uint32_t>(i);
        }
    }
    if (want_base) {
        const uint32_t m = wave_min_u32(mb);
        min_base = m == UINT32_MAX ? FLT_MAX : order_key_float(m);
    }
    const uint32_t mn = wave_min_u32(bk);
    if (mn == UINT32_MAX) return false;
    const int best = static_cast<int>(wave_min_u32(bk == mn ? bi : UINT32_MAX));
    out = f[best];
    __syncthreads();
    if (lane == 0) f[best].second |= kPoolUsed;
    __syncthreads();
    return true;
}

__device__ __forceinline__ bool pickup(Entry* f, int size, Entry& out, int lane)
{
    float unused;
    return pickup(f, size, out, lane, false, unused);
}

// XCD-aware block -> slot mapping: the dispatcher deals consecutive
// workgroups round-robin over the 8 XCDs, so block b runs on XCD b % 8.
// Slot ranges are handed out in contiguous runs per XCD, so routes sorted by
// graph group share one XCD's L2.  A bijection on [0, nblocks).
__device__ __forceinline__ uint32_t xcd_slot(uint32_t b, uint32_t nblocks)
{
    const uint32_t xcd = b & 7u;
    const uint32_t k = b >> 3;
    const uint32_t q = nblocks >> 3;
    const uint32_t r = nblocks & 7u;
    return xcd * q + (xcd < r ? xcd : r) + k;
}

}  // namespace gofann
