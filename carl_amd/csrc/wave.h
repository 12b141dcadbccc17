// wave.h - wave64 primitives: DPP prefix sum and a cooperative item loop.
//
// The per-car and per-ball candidate lists of one tick vary from a handful
// of triangles to several hundred, so a lane-per-object loop leaves most of
// a wavefront idle behind its longest list.  waveItems flattens the lists of
// all 64 lanes and hands out (owner lane, item) pairs 64 at a time.
#pragma once

#include <hip/hip_runtime.h>

namespace carl {

// Inclusive scan over the 64 lanes: Hillis-Steele inside each row of 16
// lanes with row_shr 1/2/4/8, then row_bcast:15 and row_bcast:31 carry the
// row totals across the four rows.
__device__ __forceinline__ int waveInclusiveScan(int v)
{
    v += __builtin_amdgcn_update_dpp(0, v, 0x111, 0xf, 0xf, false);  // row_shr:1
    v += __builtin_amdgcn_update_dpp(0, v, 0x112, 0xf, 0xf, false);  // row_shr:2
    v += __builtin_amdgcn_update_dpp(0, v, 0x114, 0xf, 0xf, false);  // row_shr:4
    v += __builtin_amdgcn_update_dpp(0, v, 0x118, 0xf, 0xf, false);  // row_shr:8
    v += __builtin_amdgcn_update_dpp(0, v, 0x142, 0xa, 0xf, false);  // row_bcast:15 -> rows 1,3
    v += __builtin_amdgcn_update_dpp(0, v, 0x143, 0xc, 0xf, false);  // row_bcast:31 -> rows 2,3
    return v;
}

// Calls body(owner, item, base) once for every item < count of every lane of
// the wave, with all lanes busy.  Items of one owner are visited in ascending
// order, owners in ascending lane order, 64 consecutive pairs per round; pair
// j = base + lane runs on `lane` (base is the round's first pair), so the
// items of one owner in a round sit on consecutive lanes.
// `excl` is 64 ints of LDS private to this wave.  Every lane of the wave
// must call it (count 0 for lanes without work).
template <typename Body>
__device__ __forceinline__ void waveItems(int count, int* excl, Body&& body)
{
    const int lane = (int)(threadIdx.x & 63);
    const int incl = waveInclusiveScan(count);
    const int total = __builtin_amdgcn_readlane(incl, 63);
    excl[lane] = incl - count;
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    for (int base = 0; base < total; base += 64) {
        const int j = base + lane;
        if (j < total) {
            // largest owner whose first item is <= j (it has a non-empty list)
            int o = 0;
#pragma unroll
            for (int step = 32; step > 0; step >>= 1)
                if (excl[o + step] <= j) o += step;
            body(o, j - excl[o], base);
        }
    }
}

// waveItems with a two-stage pipeline: fetch(owner, item) issues the loads of
// the next round before process(value, owner, item, base) runs on the current
// one, so each round's memory latency overlaps the previous round's work.
// Same visiting order and lane placement as waveItems.  after(last) runs on
// every lane of the wave once per round, after process.
template <typename Fetch, typename Process, typename After>
__device__ __forceinline__ void waveItemsPipelined(int count, int* excl, Fetch&& fetch, Process&& process,
                                                   After&& after)
{
    const int lane = (int)(threadIdx.x & 63);
    const int incl = waveInclusiveScan(count);
    const int total = __builtin_amdgcn_readlane(incl, 63);
    excl[lane] = incl - count;
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    auto owner = [&](int j) {
        int o = 0;
#pragma unroll
        for (int step = 32; step > 0; step >>= 1)
            if (excl[o + step] <= j) o += step;
        return o;
    };
    if (total == 0) return;
    int o = 0, q = 0;
    if (lane < total) {
        o = owner(lane);
        q = lane - excl[o];
    }
    auto cur = fetch(o, q, lane < total);
    for (int base = 0; base < total; base += 64) {
        const int jn = base + 64 + lane;
        int on = 0, qn = 0;
        if (jn < total) {
            on = owner(jn);
            qn = jn - excl[on];
        }
        auto next = fetch(on, qn, jn < total);
        if (base + lane < total) process(cur, o, q, base);
        after(base + 64 >= total);   // every lane; true after the last round
        cur = next;
        o = on;
        q = qn;
    }
}

// waveItemsPipelined with the loads of the next D rounds in flight: a ring of
// D fetched rounds, the loop unrolled by D so every slot is a register.
// Same visiting order, lane placement and hooks as waveItemsPipelined (which
// is D = 1).
template <int D, typename Fetch, typename Process, typename After>
__device__ __forceinline__ void waveItemsDeep(int count, int* excl, Fetch&& fetch, Process&& process, After&& after)
{
    const int lane = (int)(threadIdx.x & 63);
    const int incl = waveInclusiveScan(count);
    const int total = __builtin_amdgcn_readlane(incl, 63);
    excl[lane] = incl - count;
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    if (total == 0) return;
    auto locate = [&](int j, int& o, int& q) {
        o = 0;
        q = 0;
        if (j < total) {
#pragma unroll
            for (int step = 32; step > 0; step >>= 1)
                if (excl[o + step] <= j) o += step;
            q = j - excl[o];
        }
    };
    using Value = decltype(fetch(0, 0, false));
    Value buf[D];
    int os[D], qs[D];
#pragma unroll
    for (int r = 0; r < D; r++) {
        locate(r * 64 + lane, os[r], qs[r]);
        buf[r] = fetch(os[r], qs[r], r * 64 + lane < total);
    }
    for (int base = 0; base < total;) {
#pragma unroll
        for (int r = 0; r < D; r++) {
            if (base < total) {
                const Value cur = buf[r];
                const int o = os[r], q = qs[r];
                const int jn = base + D * 64 + lane;
                locate(jn, os[r], qs[r]);
                buf[r] = fetch(os[r], qs[r], jn < total);
                if (base + lane < total) process(cur, o, q, base);
                after(base + 64 >= total);   // every lane; true after the last round
                base += 64;
            }
        }
    }
}

// waveItemsPipelined for items reached through an index: index(owner, item,
// valid) loads an item's index and fetch(index, owner, valid) its data
// through it.  The index loads run Lead + 1 rounds ahead of process(value,
// owner, base) and the data loads one round ahead, so a round waits for
// neither load's full latency (the indices are small lists, the data a small
// per-index table; both stay in the caches that per-item copies of the data
// overflow).  Same visiting order, lane placement and after() hook as
// waveItemsPipelined.
template <int Lead, typename Index, typename Fetch, typename Process, typename After>
__device__ __forceinline__ void waveItemsIndexed(int count, int* excl, Index&& index, Fetch&& fetch,
                                                 Process&& process, After&& after)
{
    const int lane = (int)(threadIdx.x & 63);
    const int incl = waveInclusiveScan(count);
    const int total = __builtin_amdgcn_readlane(incl, 63);
    excl[lane] = incl - count;
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    if (total == 0) return;
    auto locate = [&](int j, int& o, int& q) {
        o = 0;
        q = 0;
        if (j < total) {
#pragma unroll
            for (int step = 32; step > 0; step >>= 1)
                if (excl[o + step] <= j) o += step;
            q = j - excl[o];
        }
    };
    // slot r of the ring holds the owner and index of round m + 1 while
    // round m (m = r mod Lead) is processed
    int ringO[Lead], ringX[Lead];
    int o0, q0;
    locate(lane, o0, q0);
    const int x0 = index(o0, q0, lane < total);
#pragma unroll
    for (int r = 0; r < Lead; r++) {
        int q;
        locate((r + 1) * 64 + lane, ringO[r], q);
        ringX[r] = index(ringO[r], q, (r + 1) * 64 + lane < total);
    }
    auto cur = fetch(x0, o0, lane < total);
    int curO = o0;
    for (int base = 0; base < total;) {
#pragma unroll
        for (int r = 0; r < Lead; r++) {
            if (base < total) {
                const int nextO = ringO[r];
                auto next = fetch(ringX[r], nextO, base + 64 + lane < total);
                const int ja = base + (Lead + 1) * 64 + lane;
                int q;
                locate(ja, ringO[r], q);
                ringX[r] = index(ringO[r], q, ja < total);
                if (base + lane < total) process(cur, curO, base);
                after(base + 64 >= total);   // every lane; true after the last round
                cur = next;
                curO = nextO;
                base += 64;
            }
        }
    }
}

// Without a per-round hook.
template <typename Fetch, typename Process>
__device__ __forceinline__ void waveItemsPipelined(int count, int* excl, Fetch&& fetch, Process&& process)
{
    waveItemsPipelined(count, excl, fetch, process, [](bool) {});
}

}  // namespace carl
