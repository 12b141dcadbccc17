// state.h - device views of the environment state and the arena.
//
// Persistent state lives in two blocks of 32-bit words, cars and simulations
// (field numbering of include/carl_amd.h), each in tiles of 64 items: field f
// of item i is word ((i / 64) * fields + f) * 64 + i % 64.  A wavefront of 64
// consecutive cars therefore reads every field as one contiguous 256-byte
// segment, and the accessors below address a field with a buffer load whose
// per-item part is one 32-bit offset shared by every field of the item and
// whose field part is a constant (immediate offset plus a constant scalar
// offset): no 64-bit address and no per-field base pointer is formed.  Cars
// of one simulation are adjacent (c = s * nCars + local).  Export and import
// convert to and from the plane layout of the C-ABI.
//
// The arena is stored per grid cell: the triangles registered in a cell are a
// contiguous run of 64-byte records (four float4, one per half cache line
// pair), so a car walks its cell with unit-stride 16-byte loads and no
// index -> vertex indirection:
//   r0 = (v0.x, v0.y, v0.z, e1.x)       e1 = v1 - v0, e2 = v2 - v0
//   r1 = (e1.y, e1.z, e2.x, e2.y)
//   r2 = (e2.z, v1.x, v1.y, v1.z)
//   r3 = (v2.x, v2.y, v2.z, bits(tri | kPlaneFlag))
#pragma once

#include <hip/hip_runtime.h>

#include "../../include/carl_amd.h"
#include "constants.h"

namespace carl {

constexpr uint32_t kPlaneFlag = 0x80000000u;  // analytic plane triangle: skipped by the car SAT

constexpr int kMaxArenaTris = 1 << 23;  // contact-search queue entries keep a triangle index in 23 bits

struct ArenaView {
    const float4* rec;       // 4 per cell reference
    const int* cellStart;    // kCells + 1 offsets into rec (in references)
    const float4* angles;    // signed edge angles per triangle (xyz)
    const float4* tri;       // 4 per triangle, by triangle index (same record layout)
    const int* cellTri;      // triangle per cell reference, ascending within a cell
    const float4* triBox;    // 4 per triangle: contact-search screening data (arena.cpp)
    const float4* triAux;    // per triangle: edge angles xyz, packed broadphase registration range
    const float4* fineRec;   // 4 per ball-grid reference (record layout)
    const float4* fineAux;   // per ball-grid reference: edge angles xyz, packed broadphase registration range
    const int* fineStart;    // kFineCells + 1 offsets into fineRec (in references)
    const int* carStart;     // kCarCells + 1 offsets into carTri
    const int* carTri;       // triangle per car-grid reference, ascending within a cell
    const float4* native;    // 4 per triangle, native mesh metadata (arena.h); null without it
};

struct Tri {
    V3 v0, v1, v2, e1, e2;
    int idx;
    bool plane;
};

DI Tri unpackTri(const float4* rec)
{
    const float4 r0 = rec[0];
    const float4 r1 = rec[1];
    const float4 r2 = rec[2];
    const float4 r3 = rec[3];
    Tri t;
    t.v0 = V3{ r0.x, r0.y, r0.z };
    t.e1 = V3{ r0.w, r1.x, r1.y };
    t.e2 = V3{ r1.z, r1.w, r2.x };
    t.v1 = V3{ r2.y, r2.z, r2.w };
    t.v2 = V3{ r3.x, r3.y, r3.z };
    const uint32_t bits = __float_as_uint(r3.w);
    t.idx = (int)(bits & ~kPlaneFlag);
    t.plane = (bits & kPlaneFlag) != 0;
    return t;
}

DI Tri loadTri(const ArenaView& a, int ref) { return unpackTri(a.rec + 4 * (size_t)ref); }
DI Tri loadTriIdx(const ArenaView& a, int idx) { return unpackTri(a.tri + 4 * (size_t)idx); }

HDI void cellOf(V3 p, int& cx, int& cy, int& cz)
{
    float x = (p.x - kArenaMin.x) / kCellX;
    float y = (p.y - kArenaMin.y) / kCellY;
    float z = (p.z - kArenaMin.z) / kCellZ;
    x = fmin_(fmax_(x, 0.f), 48.f - 1.f);
    y = fmin_(fmax_(y, 0.f), 48.f - 1.f);
    z = fmin_(fmax_(z, 0.f), 10.f - 1.f);
    cx = (int)x;
    cy = (int)y;
    cz = (int)z;
}
HDI int flatCell(int cx, int cy, int cz) { return cx + cy * kGridX + cz * kGridX * kGridY; }

// Items rounded up to whole tiles of 64, and the word of (field, item).
HDI unsigned tiledItems(int n) { return ((unsigned)n + 63u) & ~63u; }
HDI size_t tiledWord(int f, int i, int fields) { return ((size_t)(i >> 6) * fields + f) * 64 + (i & 63); }

struct Dev {
    uint32_t* car;
    uint32_t* sim;
    int nSim, nBlue, nCars, nTotal, seed;
    ArenaView arena;
    float* ballScratch;  // native arena meshes only: the balls' contacts and rows (sim_phase.h)

    // Raw buffer resources over the two blocks (dword 3: the gfx9 raw-buffer
    // format); accesses past the end read 0 and store nothing.
    DI __amdgpu_buffer_rsrc_t carRsrc() const
    {
        return __builtin_amdgcn_make_buffer_rsrc(car, 0, (int)(4u * CARL_CAR_FIELDS * tiledItems(nTotal)), 0x00020000);
    }
    DI __amdgpu_buffer_rsrc_t simRsrc() const
    {
        return __builtin_amdgcn_make_buffer_rsrc(sim, 0, (int)(4u * CARL_SIM_FIELDS * tiledItems(nSim)), 0x00020000);
    }
    static DI int itemOff(int i, int fields) { return ((i >> 6) * fields * 64 + (i & 63)) * 4; }
    DI uint32_t cw(int f, int i) const { return __builtin_amdgcn_raw_buffer_load_b32(carRsrc(), itemOff(i, CARL_CAR_FIELDS), f * 256, 0); }
    DI uint32_t sw(int f, int s) const { return __builtin_amdgcn_raw_buffer_load_b32(simRsrc(), itemOff(s, CARL_SIM_FIELDS), f * 256, 0); }
    DI void cput(int f, int i, uint32_t v) const { __builtin_amdgcn_raw_buffer_store_b32(v, carRsrc(), itemOff(i, CARL_CAR_FIELDS), f * 256, 0); }
    DI void sput(int f, int s, uint32_t v) const { __builtin_amdgcn_raw_buffer_store_b32(v, simRsrc(), itemOff(s, CARL_SIM_FIELDS), f * 256, 0); }

    DI float cf(int f, int i) const { return __uint_as_float(cw(f, i)); }
    DI int ci(int f, int i) const { return (int)cw(f, i); }
    DI V3 cv(int f, int i) const { return V3{ cf(f, i), cf(f + 1, i), cf(f + 2, i) }; }
    DI Q4 cq(int f, int i) const { return Q4{ cf(f, i), cf(f + 1, i), cf(f + 2, i), cf(f + 3, i) }; }
    DI void setf(int f, int i, float v) const { cput(f, i, __float_as_uint(v)); }
    DI void seti(int f, int i, int v) const { cput(f, i, (uint32_t)v); }
    DI void setv(int f, int i, V3 v) const { setf(f, i, v.x); setf(f + 1, i, v.y); setf(f + 2, i, v.z); }
    DI void setq(int f, int i, Q4 q) const { setf(f, i, q.x); setf(f + 1, i, q.y); setf(f + 2, i, q.z); setf(f + 3, i, q.w); }

    // A field chosen per lane: the field part joins the per-item offset, so
    // lanes with different fields still share one load instruction.
    DI uint32_t swLane(int f, int s) const
    {
        return __builtin_amdgcn_raw_buffer_load_b32(simRsrc(), itemOff(s, CARL_SIM_FIELDS) + f * 256, 0, 0);
    }

    DI float sf(int f, int s) const { return __uint_as_float(sw(f, s)); }
    DI int si(int f, int s) const { return (int)sw(f, s); }
    DI V3 sv(int f, int s) const { return V3{ sf(f, s), sf(f + 1, s), sf(f + 2, s) }; }
    DI void ssetf(int f, int s, float v) const { sput(f, s, __float_as_uint(v)); }
    DI void sseti(int f, int s, int v) const { sput(f, s, (uint32_t)v); }
    DI void ssetv(int f, int s, V3 v) const { ssetf(f, s, v.x); ssetf(f + 1, s, v.y); ssetf(f + 2, s, v.z); }
};

}  // namespace carl
