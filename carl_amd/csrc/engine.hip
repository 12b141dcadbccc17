// engine.hip - kernels, host engine and C-ABI of the MI355X CARL step engine.
//
// Tick pipeline: the reference's eleven per-tick launches plus a device scan
// (src/RLEnvironment.cu:166-211) become four kernels per tick, in the
// reference's stage order:
//   contactKernel   per car: broadphase, suspension raycast and car-arena
//                   contact search (wave-cooperative over the cell runs)
//   carArenaKernel  per car: controls, suspension, manifold and solve
//   ballKernel      per sim: episode clock, car-car pairs, ball-arena
//                   contacts, car-ball pairs, goals
//   finishKernel    per car: integrate + impulse caches / demo respawn;
//                   per sim: ball finish, then boost pads
// The simulations are split into up to four partitions, each ticked on its
// own stream.  State stays in the structure-of-arrays planes; the contact
// kernel hands the car-arena kernel a small per-car workspace (wheel hits and
// the deepest arena contact).
#include <dlfcn.h>
#include <hip/hip_ext.h>
#include <sys/stat.h>
#include <hip/hip_runtime.h>

#include <algorithm>
#include <array>
#include <climits>
#include <cstring>
#include <memory>
#include <mutex>
#include <string>
#include <vector>

#include "../../include/carl_amd.h"
#include "arena.h"
#include "envio.h"
#include "wave.h"

using namespace carl;

namespace {

thread_local std::string g_lastError;

int fail(int code, const std::string& msg)
{
    g_lastError = msg;
    return code;
}

#define HIP_TRY(expr)                                                                   \
    do {                                                                                \
        hipError_t e_ = (expr);                                                         \
        if (e_ != hipSuccess)                                                           \
            return fail(CARL_ERR_RUNTIME, std::string(#expr) + ": " + hipGetErrorString(e_)); \
    } while (0)

#define CARL_TRY(expr)                 \
    do {                               \
        const int rc_ = (expr);        \
        if (rc_ != CARL_OK) return rc_; \
    } while (0)

// ------------------------------------------------------------------ kernels

constexpr int kTickBlock = 256;
constexpr int kMaxTickStreams = 4;

// Per-tick car workspace between the contact and the car-arena kernels, 31
// 32-bit words per car: wheel hit distance, normal xyz and source per wheel,
// then the triangle of the deepest arena contact.
// kWsBest: triangle of the deepest arena contact (-1: none); kWsMan:
// that contact as a manifold point (car-local point xyz, world point xyz,
// world normal xyz, signed distance)
enum : int { kWsDist = 0, kWsNx = 4, kWsNy = 8, kWsNz = 12, kWsSrc = 16, kWsBest = 20, kWsMan = 21, kWsPlanes = 31 };

// The workspace is tiled like the persistent state (64 cars per tile, the
// planes of a tile adjacent) and accessed with buffer loads and stores.
DI __amdgpu_buffer_rsrc_t wsRsrc(const uint32_t* ws, int n)
{
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<uint32_t*>(ws), 0, (int)(4u * kWsPlanes * tiledItems(n)),
                                             0x00020000);
}
DI uint32_t wsGet(const uint32_t* ws, int n, int plane, int car)
{
    return __builtin_amdgcn_raw_buffer_load_b32(wsRsrc(ws, n), Dev::itemOff(car, kWsPlanes), plane * 256, 0);
}
DI void wsPut(uint32_t* ws, int n, int plane, int car, uint32_t v)
{
    __builtin_amdgcn_raw_buffer_store_b32(v, wsRsrc(ws, n), Dev::itemOff(car, kWsPlanes), plane * 256, 0);
}

// Where the contact phase leaves each car's wheel hits and deepest contact
// (kWsPlanes words) for the car-arena phase.  Between the phase kernels: the
// tick workspace in HBM.
struct WsHandoff {
    uint32_t* ws;
    int n;
    DI uint32_t get(int plane, int car, int) const { return wsGet(ws, n, plane, car); }
    DI void put(int plane, int car, int, uint32_t v) const { wsPut(ws, n, plane, car, v); }
};

// In the window kernel: the LDS of the wave that searched the car, since the
// lane that searches a car's contacts is the lane that runs its car-arena
// step (words kWsPlanes x 64, indexed by lane).
struct LdsHandoff {
    uint32_t* slots;
    DI uint32_t get(int plane, int, int lane) const { return slots[plane * 64 + lane]; }
    DI void put(int plane, int, int lane, uint32_t v) const { slots[plane * 64 + lane] = v; }
};

// Simulations [begin, end) of one launch: the tick runs as independent
// partitions on separate streams so the tail of one partition's kernel
// overlaps the next kernel of the other.
struct SimRange {
    int begin, end;
};

// A1: broadphase, suspension raycast and car-arena contact search of every
// car against the pre-tick poses of the arena, the other cars and the ball.
// One wave per block; the cell runs of its kContactOwners cars are searched
// by all 64 lanes together.  Fewer owners than lanes spreads the search over
// more waves: the work is latency-bound and 65536 1v1 simulations would
// otherwise leave two waves per SIMD.
constexpr int kContactBlock = 64;
static_assert(kContactOwners <= kContactBlock, "owners are lanes of the block");

// The car candidate grid's lists reach kCarGridReach uu past their cell;
// every car test stays more than 1 uu closer to the car's centre: the box's
// corners, and the wheel rays' ends (the rays start at the anchors, in the
// centre's plane, and run along the car's down axis).  The 1 uu margin covers
// the float rounding of the tests and of the centre's cell.
constexpr float sq(float x) { return x * x; }
static_assert(sq(kHalf.x) + sq(kHalf.y) + sq(kHalf.z) < sq(kCarGridReach - 1.f), "car box beyond the car grid");
static_assert(sq(kFrontX) + sq(kFrontY) + sq(kFrontRay + 1.f) < sq(kCarGridReach - 1.f), "front rays beyond the grid");
static_assert(sq(kBackX) + sq(kBackY) + sq(kBackRay + 1.f) < sq(kCarGridReach - 1.f), "back rays beyond the grid");

// the car-grid cell holding a car's centre (false outside the grid)
DI bool carGridCell(V3 c, int& cell)
{
    const float x = (c.x - kArenaMin.x) / kCarCell;
    const float y = (c.y - kArenaMin.y) / kCarCell;
    const float z = (c.z - kArenaMin.z) / kCarCell;
    if (!(x >= 0.f && x < (float)kCarX && y >= 0.f && y < (float)kCarY && z >= 0.f && z < (float)kCarZ))
        return false;
    cell = (int)x + kCarX * ((int)y + kCarY * (int)z);
    return true;
}

// What a contact search cost its lane: the candidate items its car walked
// (none for a demolished car), whether its box met the arena (a SAT hit,
// whose contact generation is the search's costliest part) and, in 1v1,
// whether the simulation's two cars were close enough for their pair test to
// go past the distance check soon.
struct WalkCost {
    int items;
    bool sat;
    bool near;
};

// The contact search of one car per lane (car, where ok) by one wave; L is
// that wave's own LDS.  Every lane of the wave calls it; it synchronises the
// wave only.  The candidates' triangle indices are loaded Lead + 1 rounds of
// 64 items ahead of the screen, their screening data one round ahead.  In
// 1v1 the cars of a simulation must sit in lanes 2i and 2i + 1.
template <int Lead, int Owners, class Handoff>
DI WalkCost contactGroup(const Dev& d, const Handoff& out, int screen, int car, bool ok, ContactLdsT<Owners>& L,
                         int lane)
{
    ok = ok && lane < Owners;
    V3 cen = kZero;
    Q4 rot{ 0.f, 0.f, 0.f, 1.f };
    Broad bp{ 0, 0, 0 };
    bool demoed = false, fine = false;
    int first = 0, count = 0;
    V3 ball = kZero;
    if (ok) {
        cen = d.cv(CARL_CAR_CEN, car);
        rot = d.cq(CARL_CAR_ROT, car);
        bp = broadphase(d, d.cv(CARL_CAR_POS, car), d.cv(CARL_CAR_VEL, car), d.cv(CARL_CAR_ANG, car), cen, rot);
        demoed = d.ci(CARL_CAR_DEMOED, car) != 0;
        if (d.nCars == 2) ball = d.sv(CARL_SIM_BALL_POS, car >> 1);
        // the shorter of two lists that both hold every triangle the car can
        // touch, in ascending triangle order: the car-grid list of the cell
        // holding the car's centre (every triangle within kCarGridReach of
        // the cell; its items count when registered in the broadphase cell),
        // and the broadphase cell's run itself.  Both orders agree on the
        // triangles that count, so the tie-breaks by triangle pick the same
        // triangle.
        int fcell;
        const bool inGrid = carGridCell(cen, fcell);
        const int fFirst = inGrid ? d.arena.carStart[fcell] : 0;
        const int fCount = inGrid ? d.arena.carStart[fcell + 1] - fFirst : 0;
        fine = inGrid && fCount < bp.count;
        first = fine ? fFirst : bp.start;
        count = fine ? fCount : bp.count;
    }
    contactPrepare(L, lane, ok && !demoed, cen, rot, first, fine, bp.cell, screen != 0);
    waveSync();
    waveItemsIndexed<Lead>(
        count, L.excl, [&](int o, int q, bool valid) { return contactIndex(d, L, o, q, valid); },
        [&](int tri, int o, bool valid) { return contactFetchTri(d, L, tri, o, valid); },
        [&](const RefBox& b, int o, int) { contactScreen(L, b, o, lane); },
        [&](bool last) { contactDrain(d, L, lane, last); });
    waveSync();
    const bool satHit = ok && lane < Owners && L.satHits[lane] > 0;
    // 1v1: the other car of an owner's simulation is the neighbouring lane's
    // owner (owner groups start at even cars and end at even ones), so its
    // pre-tick box and flag come from that lane's registers, and the ball's
    // position was loaded with the owner's own words: the wheel rays at the
    // bodies wait for no load
    V3 ocen = kZero;
    Q4 orot{ 0.f, 0.f, 0.f, 1.f };
    bool odemoed = true;
    if (d.nCars == 2) {
        ocen = V3{ __shfl_xor(cen.x, 1), __shfl_xor(cen.y, 1), __shfl_xor(cen.z, 1) };
        orot = Q4{ __shfl_xor(rot.x, 1), __shfl_xor(rot.y, 1), __shfl_xor(rot.z, 1), __shfl_xor(rot.w, 1) };
        odemoed = __shfl_xor((int)demoed, 1) != 0;
    }
    Wheels w;
    int best = -1;
    float pt[10] = {};
    if (ok) {
        if (d.nCars == 2)
            best = contactFinishWith(L, lane, cen, rot, w, [&](const V3* start, V3 dir, Wheels& ww) {
                if (!odemoed && !(lensq(ocen - cen) > kCarRayReach * kCarRayReach))
                    raycastCar(start, dir, ocen, orot, ww);
                if (!(lensq(ball - cen) > kBallRayReach * kBallRayReach)) raycastBall(start, dir, ball, ww);
            });
        else
            best = contactFinish(d, L, lane, car, car / d.nCars, cen, rot, w);
        if (best >= 0) {
#pragma unroll
            for (int i = 0; i < 10; i++) pt[i] = L.bestPt[i][lane];
        }
    }
    // every lane's reads of the search area come before any lane's handoff
    // writes (an LDS handoff may share that area)
    waveSync();
    if (!ok) return WalkCost{ 0, false, false };
    // two car boxes within twice the box diagonal of each other (the pair
    // test's distance bound), with the travel of a window on top
    const float near = 4.f * len(kHalf);
    const WalkCost cost{ demoed ? 0 : count, satHit,
                         d.nCars == 2 && !demoed && !odemoed && lensq(ocen - cen) < near * near };
#pragma unroll
    for (int k = 0; k < kWheels; k++) {
        out.put(kWsDist + k, car, lane, __float_as_uint(w.dist[k]));
        out.put(kWsNx + k, car, lane, __float_as_uint(w.normal[k].x));
        out.put(kWsNy + k, car, lane, __float_as_uint(w.normal[k].y));
        out.put(kWsNz + k, car, lane, __float_as_uint(w.normal[k].z));
        out.put(kWsSrc + k, car, lane, (uint32_t)w.src[k]);
    }
    out.put(kWsBest, car, lane, (uint32_t)best);
    if (best >= 0) {
#pragma unroll
        for (int i = 0; i < 10; i++) out.put(kWsMan + i, car, lane, __float_as_uint(pt[i]));
    }
    return cost;
}

__global__ __launch_bounds__(kContactBlock) void contactKernel(Dev d, uint32_t* __restrict__ ws, int screen, SimRange range)
{
    __shared__ ContactLds L;
    const int car = range.begin * d.nCars + blockIdx.x * kContactOwners + (int)threadIdx.x;
    contactGroup<1, kContactOwners>(d, WsHandoff{ ws, d.nTotal }, screen, car, car < range.end * d.nCars, L,
                                    threadIdx.x);
}

// A2: controls, car-arena contacts, suspension and the contact solve.
// two waves per SIMD keep all of its waves resident at 65536 1v1 simulations
template <class Handoff>
DI void carArenaCar(const Dev& d, const Handoff& in, int kind, const void* __restrict__ actions, int tick, int car,
                    int lane)
{
    Wheels w;
#pragma unroll
    for (int k = 0; k < kWheels; k++) {
        w.dist[k] = __uint_as_float(in.get(kWsDist + k, car, lane));
        w.normal[k] = V3{ __uint_as_float(in.get(kWsNx + k, car, lane)), __uint_as_float(in.get(kWsNy + k, car, lane)),
                          __uint_as_float(in.get(kWsNz + k, car, lane)) };
        w.src[k] = (int)in.get(kWsSrc + k, car, lane);
    }
    const int best = (int)in.get(kWsBest, car, lane);
    ManPt bestPt{};
    if (best >= 0) {
        float v[10];
#pragma unroll
        for (int i = 0; i < 10; i++) v[i] = __uint_as_float(in.get(kWsMan + i, car, lane));
        bestPt = ManPt{ V3{ v[0], v[1], v[2] }, V3{ v[3], v[4], v[5] }, V3{ v[6], v[7], v[8] }, v[9] };
    }
    const Controls ctl = decodeControls(kind, actions, car);
    const bool demoed = d.ci(CARL_CAR_DEMOED, car) != 0;
    CarRegs r;
    loadRegs(d, car, r);
    storeWheelOutputs(d, car, w);
    d.setf(CARL_CAR_CTRL_THROTTLE, car, ctl.throttle);
    d.setf(CARL_CAR_CTRL_STEER, car, ctl.steer);
    d.setf(CARL_CAR_CTRL_YAW, car, ctl.yaw);
    d.setf(CARL_CAR_CTRL_PITCH, car, ctl.pitch);
    d.setf(CARL_CAR_CTRL_ROLL, car, ctl.roll);
    d.seti(CARL_CAR_CTRL_JUMP, car, ctl.jump);
    d.seti(CARL_CAR_CTRL_BOOST, car, ctl.boost);
    d.seti(CARL_CAR_CTRL_SLIDE, car, ctl.slide);
    if (demoed) return;
    applyControls(r, ctl, w);
    solveCarArena(r, w, best >= 0, bestPt, tick);
    storeRegs(d, car, r);
}

__global__ __launch_bounds__(kTickBlock, 2) void carArenaKernel(Dev d, const uint32_t* __restrict__ ws, int kind,
                                                             const void* __restrict__ actions, int tick,
                                                             SimRange range)
{
    const int car = range.begin * d.nCars + blockIdx.x * kTickBlock + threadIdx.x;
    if (car < range.end * d.nCars)
        carArenaCar(d, WsHandoff{ const_cast<uint32_t*>(ws), d.nTotal }, kind, actions, tick, car, (int)threadIdx.x & 63);
}

// Episode clock and the car-car pairs of one simulation, (b, a) with b the
// later car (Kernels.cu:42-55, CarCar/Solve.cuh:63-151).
DI void carCarSim(const Dev& d, int sim, int tick)
{
    d.sseti(CARL_SIM_EPISODE_TICKS, sim, d.si(CARL_SIM_EPISODE_TICKS, sim) + 1);
    const int base = sim * d.nCars;
    for (int a = 0; a < d.nCars - 1; a++)
        for (int b = a + 1; b < d.nCars; b++) carCarPair(d, base + b, base + a, tick);
}

// B: per simulation the episode clock and the car-car pairs, then ball-arena
// contacts, car-ball pairs and goal detection (the reference's
// carCarBallSolveKernel, Kernels.cu:162-172).  One wave per block; the arena
// contacts of its kBallOwners balls are gathered by all 64 lanes
// cooperatively.  The car-car solve of a colliding pair is a long serial
// chain on one lane: inside this kernel it delays only its own wave, where a
// kernel of its own would end only when that chain ends.
constexpr int kBallBlock = 64;
constexpr int kBallOwners = 32;

// One simulation per lane of the first kBallOwners (sim, where ok) by one
// wave; L is that wave's own LDS.  Every lane of the wave calls it; it
// synchronises the wave only.  With Native (arena metadata) each owner lane
// gathers and solves its ball against the native meshes alone.
template <bool Native>
DI void ballGroup(const Dev& d, int tick, int sim, bool ok, BallLds& L, int lane)
{
    ok = ok && lane < kBallOwners;
    if constexpr (Native) {
        if (ok) {
            carCarSim(d, sim, tick);
            nativeBallTick(d, sim, tick);
        }
        return;
    }
    if (ok) carCarSim(d, sim, tick);
    const bool awake = ok && !ballSleeping(d, sim);
    const V3 center = ok ? d.sv(CARL_SIM_BALL_POS, sim) : kZero;
    int items = 0, first = 0, cell = 0;
    bool sequential = false;
    if (awake) {
        if (ballGridCell(center, cell)) {
            first = d.arena.fineStart[cell];
            items = d.arena.fineStart[cell + 1] - first;
        } else {
            sequential = true;
        }
    }
    ballPrepare(L, lane, center, first);
    waveSync();
    BallContact cs[4];
#pragma unroll
    for (int k = 0; k < 4; k++) cs[k] = BallContact{ kZero, kZero, kZero, 0.f, kZero };
    int count = 0;
    bool hit = false;
    int roundBase = 0;
    waveItemsPipelined(
        items, L.excl, [&](int o, int q, bool valid) { return ballGatherFetch(d, L, o, q, valid); },
        [&](const BallItem& item, int o, int, int) { hit = ballGatherItem(L, item, o, lane); },
        [&](bool) {
            __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
            __builtin_amdgcn_wave_barrier();
            __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
            const unsigned long long hits = __ballot(hit);
            hit = false;
            if (items > 0) {
                const int a = L.excl[lane] - roundBase, b = L.excl[lane] + items - roundBase;
                if (b > 0 && a < 64) foldStashedContacts(L, hits, a > 0 ? a : 0, b < 64 ? b : 64, cs, count);
            }
            roundBase += 64;
            __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
            __builtin_amdgcn_wave_barrier();
            __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
        });
    if (!ok) return;
    if (sequential) count = gatherBallContacts(d, center, cs);
    ballTick(d, sim, tick, cs, count);
}

__global__ __launch_bounds__(kBallBlock) void ballKernel(Dev d, int tick, SimRange range)
{
    __shared__ BallLds L;
    const int sim = range.begin + blockIdx.x * kBallOwners + (int)threadIdx.x;
    ballGroup<false>(d, tick, sim, sim < range.end, L, threadIdx.x);
}

// the same with the native arena meshes
__global__ __launch_bounds__(kBallBlock) void ballNativeKernel(Dev d, int tick, SimRange range)
{
    __shared__ BallLds L;
    const int sim = range.begin + blockIdx.x * kBallOwners + (int)threadIdx.x;
    ballGroup<true>(d, tick, sim, sim < range.end, L, threadIdx.x);
}

// C + D: integration and impulse caches of every car and ball, then the
// boost pads of each simulation once all of its cars have moved.  A block
// owns whole simulations (simsPerBlock * nCars car lanes).
__global__ __launch_bounds__(kTickBlock) void finishKernel(Dev d, int simsPerBlock, SimRange range)
{
    const int t = threadIdx.x;
    const int simBase = range.begin + blockIdx.x * simsPerBlock;
    const int mySim = simBase + t / d.nCars;
    const int car = mySim * d.nCars + t % d.nCars;
    const int laneSim = simBase + t;
    if (t < simsPerBlock * d.nCars && mySim < range.end) finishCar(d, car);
    const bool simOk = t < simsPerBlock && laneSim < range.end;
    if (simOk) finishBall(d, laneSim);
    __syncthreads();
    if (simOk) boostPads(d, laneSim);
}

// The whole tick window in one launch: a block owns simulations
// [begin + blockIdx.x * simsPerBlock, +simsPerBlock) and runs every phase of
// every tick on them, with block barriers between the phases.  Simulations
// share nothing but the read-only arena, so no other block is ever waited
// for: a slow wave holds up its own block, not a grid-wide kernel boundary.
// Two-wave blocks (four per CU) wait less at the phase barriers than
// four-wave blocks at the same occupancy (measured +1.7% per step), and
// measured 1-3% faster than one-wave blocks of 32 simulations, whose
// barriers cost nothing.
#ifndef CARL_WINDOW_BLOCK
#define CARL_WINDOW_BLOCK 128
#endif
#ifndef CARL_WINDOW_SIMS
#define CARL_WINDOW_SIMS 64
#endif
constexpr int kWindowBlock = CARL_WINDOW_BLOCK;
constexpr int kWindowWaves = kWindowBlock / 64;
constexpr int kDefaultWindowSims = CARL_WINDOW_SIMS;
constexpr int kAutoWindowMin = 8;   // smallest automatic window workgroup (simulations)
// rounds of candidate-index loads the window kernel's contact search keeps in
// flight beyond the round of screening-data loads
#ifndef CARL_WINDOW_CONTACT_LEAD
#define CARL_WINDOW_CONTACT_LEAD 1
#endif
constexpr int kWindowContactLead = CARL_WINDOW_CONTACT_LEAD;
// cars whose contacts one wave of the window kernel searches together
#ifndef CARL_WINDOW_CONTACT_OWNERS
#define CARL_WINDOW_CONTACT_OWNERS 64
#endif
constexpr int kWindowContactOwners = CARL_WINDOW_CONTACT_OWNERS;

// Each wave has an LDS area of its own, used by its contact search, then by
// the contact results it hands to the car-arena phase, and in the ball phase
// by its ball gather (the phases of one wave never overlap, and no wave
// touches another wave's area).  With a whole wave of
// contact owners that is 19.7 KB per wave, 39.4 KB per workgroup: four
// workgroups per CU, the occupancy the 256-VGPR budget allows.  The phases are
// still separated by workgroup barriers: a phase reads state words other
// threads of the workgroup wrote in the phase before.
union WaveLds {
    ContactLdsT<kWindowContactOwners> contact;
    uint32_t hand[kWsPlanes * 64];   // the contact phase's results, read by the car-arena phase
    BallLds ball;
};
// Car car0 + 64 w + l is contact owner l of wave w and car-arena thread
// 64 w + l: a block holds at most kWindowBlock cars, one contact group per
// wave, so each car's handoff stays in the lane that produced it.
static_assert(kWindowContactOwners == 64, "the LDS handoff pairs contact owners with car-arena threads");
struct WindowLds {
    WaveLds wave[kWindowWaves];
};
static_assert(4 * sizeof(WindowLds) <= 160 * 1024, "four window workgroups per CU");

// Phases of a tick in the window kernel, timed by the stage profile.
enum WindowStage { kStageContact, kStageCarArena, kStageBall, kStageFinish, kStagePads, kWindowStages };
static_assert(kWindowStages == CARL_STAGES && kStagePads == CARL_STAGE_PADS, "stage ids of the C-ABI");

// Stage-profile counters (64-bit wall-clock ticks), summed over launches
// except the three per-launch words, which the last workgroup of a launch
// to finish resets (kProfFirst to all ones, the others to zero).
enum ProfWord {
    kProfStages = 0,                      // [stage]: all workgroups' time in the stage
    kProfLast = kProfStages + kWindowStages,  // [stage]: the stages of each launch's last workgroup
    kProfLastDelay = kProfLast + kWindowStages,  // that workgroup's start after the launch's first start
    kProfSpan,                            // first workgroup start to last workgroup end
    kProfFirst,                           // per launch: earliest workgroup start
    kProfEnd,                             // per launch: latest workgroup end
    kProfDone,                            // per launch: workgroups finished
    kProfWords
};

// Balanced 1v1 and 2v2 launches deal the simulations to the workgroups in
// units of kUnitCars cars (dealUnitSims consecutive simulations): slot s
// of workgroup b (wave 2 b + s / kWaveUnits) holds one unit, its cars in
// kUnitCars consecutive lanes and its balls in as many lanes as it has
// simulations.  Simulations share nothing, so the deal changes no result; it
// is made so that the workgroups finish together.  A unit's cars fill whole
// 128-byte lines of every car field (1v1 units of 8 simulations left half
// lines to workgroups on other XCDs, whose L2s then fetched the same lines:
// the launch read 2.5 times the bytes).
//
// The deal needs no pass of its own.  At its last tick every launch files
// each unit under the class of its cost (dealClass) in an output list: one
// atomic per unit on a count, then the unit at that position of the list.
// Each class has kDealSubs lists, unit u going to list u % kDealSubs, so
// that units of equal cost (the kickoffs, early on) do not all wait on one
// count.  The next launch reads the lists back in rank order, costliest
// class first (any order within a class), and deals them to the
// waves in rounds: round 0 gives the costliest units, one to each wave in
// order; every later round gives its units in reverse order, so that the
// waves holding the costliest units get the cheapest of each round (the
// costs have a long tail: a car whose box meets the arena every tick, a pair
// that may collide).  Two units of pairs that may collide thus fall to the
// two waves of one workgroup, whose pair solves run side by side.  Three
// list sets rotate: launch L reads set L % 3, files into set (L + 1) % 3
// (cleared by launch L - 1) and clears the counts of set (L + 2) % 3, which
// no launch touches again before L + 1.
constexpr int kUnitCars = 32;                            // one 128-byte line of each car field
constexpr int kUnitSlots = 4;                            // units per balanced workgroup
constexpr int kWaveUnits = kUnitSlots / 2;               // units per wave
// simulations per unit and per balanced workgroup, by cars per simulation
// (0: no balanced launch)
HDI constexpr int dealUnitSims(int cars) { return cars == 2 || cars == 4 ? kUnitCars / cars : 0; }
HDI constexpr int dealBlockSims(int cars) { return kUnitSlots * dealUnitSims(cars); }
constexpr int kDealClasses = 32;
constexpr int kDealSubs = 4;
constexpr int kDealLists = kDealClasses * kDealSubs;
constexpr int kListsPerThread = kDealLists / 128;   // of a balanced workgroup's threads, in the deal's scan
constexpr int kDealSets = 3;
// A unit's cost is its contact work in the launch's last tick, in candidate
// items (each about 0.04 us of its wave's time).  A car whose box met the
// arena costs its wave about 6 us of contact generation (160 items),
// counted at half, kSatCost, since it persists less from one launch to the
// next than a candidate count does; a pair that may collide (cars within
// twice their box diagonal) costs about 25 us per tick of its serial solve,
// kPairCost items.  (The cost summed over the launch's ticks ranked the
// units no better.)
constexpr int kSatCost = 80;
constexpr int kPairCost = 720;

// cost class: four classes per doubling from 8 items up (class 0 below)
DI int dealClass(int cost)
{
    if (cost < 8) return 0;
    return min(kDealClasses - 1, 1 + (int)(4.f * __log2f((float)cost * (1.f / 8.f))));
}

// list k = kDealSubs c + j of a set holds up to nUnits / kDealSubs units
// from outList + k nUnits / kDealSubs, its count at outCount[k]
struct WindowMap {
    const int* inCount;   // the deal's counts and lists (null: slot s of workgroup b holds unit 4 b + s)
    const int* inList;
    int* outCount;        // this launch's filing
    int* outList;
    int* clearCount;      // the counts the next launch files into
    int nUnits;
};

// The window kernel's body.  With Profile, thread 0 of each workgroup reads
// the wall clock (the constant-rate counter) at the start and after every
// phase barrier; a phase's time runs from the barrier before it to its own,
// barrier wait included.  At the end each workgroup adds its phase times to
// the kProfStages sums, and the launch's last workgroup to finish adds its
// own phase times, its start delay and the launch's span.  Without Profile
// the code is the plain kernel.
template <bool Profile, bool Native, int Cars, bool Balanced>
DI void tickWindowBody(Dev d0, uint32_t* __restrict__ ws, int screen, int kind, const void* __restrict__ actions,
                       int tick0, int ticks, int simsPerBlock, SimRange range, WindowMap map,
                       unsigned long long* __restrict__ prof)
{
    static_assert(!Balanced || dealUnitSims(Cars) > 0, "balanced launches are 1v1 or 2v2");
    constexpr int kUnitSims = Balanced ? dealUnitSims(Cars) : 1, kBlockSims = kUnitSlots * kUnitSims;
    static_assert(kWindowBlock == 2 * 64 && kWaveUnits * kUnitCars == 64 && kWaveUnits * kUnitSims <= kBallOwners,
                  "a balanced wave holds kWaveUnits units: 64 cars, at most kBallOwners balls");
    // a fixed car count (Cars > 0) lets every per-simulation loop fold
    Dev d = d0;
    if constexpr (Cars > 0) d.nCars = Cars;
    __shared__ WindowLds L;
    __shared__ int unit[Balanced ? kUnitSlots : 1];
    const int t = threadIdx.x, wave = t >> 6, lane = t & 63;
    // balanced: the car of thread (or contact owner) i, the simulation of
    // workgroup position j (ball owners, finish and pads)
    auto slotCar = [&](int i) { return unit[i / kUnitCars] * kUnitCars + i % kUnitCars; };
    auto slotSim = [&](int j) { return unit[j / kUnitSims] * kUnitSims + j % kUnitSims; };
    if constexpr (Balanced) {
        if (map.inCount) {
            // the lists' first ranks, costliest class first, in the LDS the
            // contact phase takes over afterwards; each thread scans
            // kListsPerThread of them: lists k in rank order hold class
            // kDealClasses - 1 - k / kDealSubs
            static_assert(kListsPerThread * kWindowBlock == kDealLists && kDealLists * sizeof(int) <= sizeof(WaveLds),
                          "the deal's scan: whole lists per thread, in one wave's LDS");
            int* first = reinterpret_cast<int*>(&L.wave[0]);
            __shared__ int waveSum[kWindowWaves];
            int n[kListsPerThread], sum = 0;
#pragma unroll
            for (int i = 0; i < kListsPerThread; i++) {
                const int k = kListsPerThread * t + i;
                n[i] = map.inCount[(kDealClasses - 1 - k / kDealSubs) * kDealSubs + k % kDealSubs];
                sum += n[i];
            }
            int incl = sum;
            for (int o = 1; o < 64; o <<= 1) {
                const int y = __shfl_up(incl, o);
                if (lane >= o) incl += y;
            }
            if (lane == 63) waveSum[wave] = incl;
            __syncthreads();
            int r = incl - sum;
            for (int v = 0; v < wave; v++) r += waveSum[v];
#pragma unroll
            for (int i = 0; i < kListsPerThread; i++) {
                first[kListsPerThread * t + i] = r;
                r += n[i];
            }
            __syncthreads();
            if (t < kUnitSlots) {
                const int waves = map.nUnits / kWaveUnits, wv = 2 * blockIdx.x + t / kWaveUnits, r = t % kWaveUnits;
                const int rank = r == 0 ? wv : r * waves + (waves - 1 - wv);
                // the last list whose first rank is at most rank
                int lo = 0;
                for (int step = kDealLists / 2; step > 0; step >>= 1)
                    if (lo + step < kDealLists && first[lo + step] <= rank) lo += step;
                const int per = map.nUnits / kDealSubs;
                const int k = (kDealClasses - 1 - lo / kDealSubs) * kDealSubs + lo % kDealSubs;
                unit[t] = map.inList[(size_t)k * per + min(rank - first[lo], per - 1)];
            }
            __syncthreads();   // the scan's LDS is the contact phase's
        } else if (t < kUnitSlots) {
            unit[t] = blockIdx.x * kUnitSlots + t;
        }
        if (blockIdx.x == 0) {
#pragma unroll
            for (int i = 0; i < kListsPerThread; i++) map.clearCount[kListsPerThread * t + i] = 0;
        }
        __syncthreads();
    }
    const int sim0 = range.begin + blockIdx.x * simsPerBlock;
    const int simEnd = min(sim0 + simsPerBlock, range.end);
    const int car0 = sim0 * d.nCars, carEnd = simEnd * d.nCars;
    unsigned long long acc[kWindowStages] = {}, first = 0, last = 0;
    auto mark = [&](int stage) {
        if constexpr (Profile) {
            if (t == 0) {
                const unsigned long long now = wall_clock64();
                acc[stage] += now - last;
                last = now;
            }
        }
    };
    if constexpr (Profile) {
        if (t == 0) first = last = wall_clock64();
    }
    for (int k = 0; k < ticks; k++) {
        const int tick = tick0 + k;
        if constexpr (Balanced) {
            const WalkCost c = contactGroup<kWindowContactLead, kWindowContactOwners>(
                d, LdsHandoff{ L.wave[wave].hand }, screen, slotCar(t), true, L.wave[wave].contact, lane);
            if (k == ticks - 1) {
                // the unit's cost for the next deal (a pair counted at its first car)
                int w = c.items + (c.sat ? kSatCost : 0) + (c.near && (lane & 1) == 0 ? kPairCost : 0);
                for (int o = kUnitCars / 2; o > 0; o >>= 1) w += __shfl_xor(w, o);
                if (lane % kUnitCars == 0) {
                    const int u = unit[t / kUnitCars], l = dealClass(w) * kDealSubs + u % kDealSubs;
                    map.outList[(size_t)l * (map.nUnits / kDealSubs) + atomicAdd(&map.outCount[l], 1)] = u;
                }
            }
        } else {
            for (int g = car0 + wave * kWindowContactOwners; g < carEnd; g += kWindowWaves * kWindowContactOwners)
                contactGroup<kWindowContactLead, kWindowContactOwners>(d, LdsHandoff{ L.wave[wave].hand }, screen,
                                                                         g + lane, g + lane < carEnd,
                                                                         L.wave[wave].contact, lane);
        }
        __syncthreads();
        mark(kStageContact);
        if constexpr (Balanced) {
            carArenaCar(d, LdsHandoff{ L.wave[wave].hand }, kind, actions, tick, slotCar(t), lane);
        } else {
            for (int c = car0 + t; c < carEnd; c += kWindowBlock)
                carArenaCar(d, LdsHandoff{ L.wave[wave].hand }, kind, actions, tick, c, lane);
        }
        __syncthreads();
        mark(kStageCarArena);
        if constexpr (Balanced) {
            constexpr int kWaveSims = kWaveUnits * kUnitSims;
            ballGroup<Native>(d, tick, slotSim(kWaveSims * wave + lane % kWaveSims), lane < kWaveSims,
                              L.wave[wave].ball, lane);
        } else {
            // the block's simulations split evenly between the waves (a
            // block of 21 3v3 or 32 2v2 simulations would otherwise leave
            // the second wave idle): at most kBallOwners per wave and group
            const int per = (simEnd - sim0 + kWindowWaves - 1) / kWindowWaves;
            const int wEnd = min(sim0 + (wave + 1) * per, simEnd);
            for (int g = sim0 + wave * per; g < wEnd; g += kBallOwners)
                ballGroup<Native>(d, tick, g + lane, g + lane < wEnd, L.wave[wave].ball, lane);
        }
        __syncthreads();
        mark(kStageBall);
        if constexpr (Balanced) {
            finishCar(d, slotCar(t));
            if (t < kBlockSims) finishBall(d, slotSim(t));
        } else {
            for (int c = car0 + t; c < carEnd; c += kWindowBlock) finishCar(d, c);
            for (int s = sim0 + t; s < simEnd; s += kWindowBlock) finishBall(d, s);
        }
        __syncthreads();
        mark(kStageFinish);
        if constexpr (Balanced) {
            int tp = t;
            asm volatile("" : "+v"(tp));
            constexpr int kParts = kWindowBlock / kBlockSims;   // pad ranges per simulation
            const int q = tp / kBlockSims, j = tp - q * kBlockSims;
            if constexpr (kParts == kWindowWaves && Cars > 0) {
                // one pad range per wave (1v1), fixed at compile time: each
                // wave loads only its own pads' cooldowns (1,000-step bench:
                // pad phase 5.0 -> 4.4 us per tick)
                static_assert(kPads % 2 == 0, "two equal pad ranges");
                if (__builtin_amdgcn_readfirstlane(wave) == 0)
                    boostPadsRangeT<Cars, 0, kPads / 2>(d, slotSim(j), 0, kPads / 2);
                else
                    boostPadsRangeT<Cars, kPads / 2, kPads>(d, slotSim(j), kPads / 2, kPads);
            } else {
                boostPadsSpan(d, slotSim(j), kPads * q / kParts, kPads * (q + 1) / kParts, kParts);
            }
        } else {
            // boost pads: the workgroup's threads split into kWindowBlock /
            // simsPerBlock parts, each taking a contiguous range of every
            // simulation's pads (in 1v1 two parts, one wave each).  The
            // split is derived here from a copy of the thread index that the
            // optimiser cannot hoist, so it holds no registers through the
            // other phases.
            int tp = t;
            asm volatile("" : "+v"(tp));
            const int parts = kWindowBlock / simsPerBlock, q = tp / simsPerBlock, j = tp - q * simsPerBlock;
            if (parts == kWindowWaves) {
                // one range per wave (at most two cars per simulation): fixed
                // at compile time, as in dealt 1v1 launches
                if (j < simEnd - sim0) {
                    if (__builtin_amdgcn_readfirstlane(wave) == 0)
                        boostPadsRangeT<2, 0, kPads / 2>(d, sim0 + j, 0, kPads / 2);
                    else
                        boostPadsRangeT<2, kPads / 2, kPads>(d, sim0 + j, kPads / 2, kPads);
                }
            } else if (q < parts && j < simEnd - sim0) {
                boostPadsSpan(d, sim0 + j, kPads * q / parts, kPads * (q + 1) / parts, parts);
            }
        }
        __syncthreads();
        mark(kStagePads);
    }
    if constexpr (Profile) {
        if (t == 0) {
            for (int st = 0; st < kWindowStages; st++) atomicAdd(&prof[kProfStages + st], acc[st]);
            atomicMin(&prof[kProfFirst], first);
            atomicMax(&prof[kProfEnd], last);
            __threadfence();
            if (atomicAdd(&prof[kProfDone], 1ull) == gridDim.x - 1) {
                // every other workgroup has published its start and end
                __threadfence();
                const unsigned long long first0 = atomicMin(&prof[kProfFirst], ~0ull);
                const unsigned long long end1 = atomicMax(&prof[kProfEnd], 0ull);
                for (int st = 0; st < kWindowStages; st++) atomicAdd(&prof[kProfLast + st], acc[st]);
                atomicAdd(&prof[kProfLastDelay], first - first0);
                atomicAdd(&prof[kProfSpan], end1 - first0);
                atomicExch(&prof[kProfFirst], ~0ull);
                atomicExch(&prof[kProfEnd], 0ull);
                atomicExch(&prof[kProfDone], 0ull);
            }
        }
    }
}

// two waves per SIMD (the second bound is waves per execution unit): 256
// VGPRs.  Cars > 0: instantiated for that many cars per simulation (1v1, the
// common case, measured 6% faster than the same kernel with the count
// read at run time; 2v2 and 3v3 5% and 3%); 0: any count.  Balanced: the
// 1v1 instance that takes its simulations from the deal (WindowMap).
template <int Cars, bool Balanced>
__global__ __launch_bounds__(kWindowBlock, 2) void tickWindowKernel(Dev d, uint32_t* __restrict__ ws, int screen,
                                                                 int kind, const void* __restrict__ actions,
                                                                 int tick0, int ticks, int simsPerBlock,
                                                                 SimRange range, WindowMap map)
{
    tickWindowBody<false, false, Cars, Balanced>(d, ws, screen, kind, actions, tick0, ticks, simsPerBlock, range,
                                                 map, nullptr);
}

using WindowKernel = void (*)(Dev, uint32_t*, int, int, const void*, int, int, int, SimRange, WindowMap);

// the instance for a car count: 1v1, 2v2 and 3v3 have their own
WindowKernel windowKernelFor(int nCars, bool balanced)
{
    switch (nCars) {
    case 2: return balanced ? tickWindowKernel<2, true> : tickWindowKernel<2, false>;
    case 4: return balanced ? tickWindowKernel<4, true> : tickWindowKernel<4, false>;
    case 6: return tickWindowKernel<6, false>;
    default: return tickWindowKernel<0, false>;
    }
}

// the same with the native arena meshes
__global__ __launch_bounds__(kWindowBlock, 2) void tickWindowNativeKernel(Dev d, uint32_t* __restrict__ ws,
                                                                       int screen, int kind,
                                                                       const void* __restrict__ actions, int tick0,
                                                                       int ticks, int simsPerBlock, SimRange range,
                                                                       WindowMap map)
{
    tickWindowBody<false, true, 0, false>(d, ws, screen, kind, actions, tick0, ticks, simsPerBlock, range, map,
                                          nullptr);
}

// the same kernel with the stage profile
template <int Cars, bool Balanced>
__global__ __launch_bounds__(kWindowBlock, 2) void tickWindowProfileKernel(Dev d, uint32_t* __restrict__ ws,
                                                                        int screen, int kind,
                                                                        const void* __restrict__ actions, int tick0,
                                                                        int ticks, int simsPerBlock, SimRange range,
                                                                        WindowMap map,
                                                                        unsigned long long* __restrict__ prof)
{
    tickWindowBody<true, false, Cars, Balanced>(d, ws, screen, kind, actions, tick0, ticks, simsPerBlock, range,
                                                map, prof);
}

using ProfileKernel = void (*)(Dev, uint32_t*, int, int, const void*, int, int, int, SimRange, WindowMap,
                               unsigned long long*);

// the profiled twin of windowKernelFor's instance for a car count
ProfileKernel profileKernelFor(int nCars, bool balanced)
{
    switch (nCars) {
    case 2: return balanced ? tickWindowProfileKernel<2, true> : tickWindowProfileKernel<2, false>;
    case 4: return balanced ? tickWindowProfileKernel<4, true> : tickWindowProfileKernel<4, false>;
    case 6: return tickWindowProfileKernel<6, false>;
    default: return tickWindowProfileKernel<0, false>;
    }
}

__global__ void resetKernel(Dev d, int nOrange)
{
    const int s = blockIdx.x * blockDim.x + threadIdx.x;
    if (s < d.nSim) fullResetSim(d, s, nOrange);
}

__global__ void resetDonesKernel(Dev d, int nOrange, int tickCount, DoneRule rule)
{
    const int s = blockIdx.x * blockDim.x + threadIdx.x;
    if (s < d.nSim) resetAfterDone(d, s, tickCount, rule, nOrange);
}

__global__ void rewardsDonesKernel(Dev d, int tickCount, DoneRule rule, float* rewards, bool* dones, int* tScore,
                                   int* tTicks, bool* tOvertime)
{
    const int s = blockIdx.x * blockDim.x + threadIdx.x;
    if (s >= d.nSim) return;
    rewards[s] = (float)d.si(CARL_SIM_LAST_SCORER, s);
    dones[s] = simDone(d, s, tickCount, rule);
    tScore[s] = d.si(CARL_SIM_BLUE_SCORE, s) - d.si(CARL_SIM_ORANGE_SCORE, s);
    tTicks[s] = d.si(CARL_SIM_EPISODE_TICKS, s);
    tOvertime[s] = d.si(CARL_SIM_OVERTIME, s) != 0;
}

__global__ void matchKernel(Dev d, int* score, int* ticks, bool* overtime, const bool* mask, const int* list,
                            const int* count)
{
    int s = blockIdx.x * blockDim.x + threadIdx.x;
    if (list) {
        if (s >= *count) return;
        s = list[s];
    }
    if (s >= d.nSim || (mask && !mask[s])) return;
    score[s] = d.si(CARL_SIM_BLUE_SCORE, s) - d.si(CARL_SIM_ORANGE_SCORE, s);
    ticks[s] = d.si(CARL_SIM_EPISODE_TICKS, s);
    overtime[s] = d.si(CARL_SIM_OVERTIME, s) != 0;
}

// Row-major outputs (observations, canonical states) are written through
// LDS.  A packing workgroup is four waves; rows go in chunks of up to 64, and
// wave q builds column part q (packObservationPart / packStatePart) of every
// row of the chunk, one row per lane, at an odd stride so the lanes' writes
// fall in distinct banks.  The workgroup then stores the chunk's rows as one
// contiguous run, so each store instruction covers consecutive words (a lane
// storing its own row touched a different line per lane and per store).
constexpr int kPackBlock = 64 * kRowParts;
constexpr int kPackLdsBytes = 38 * 1024;   // four workgroups per CU

HDI int packStride(int rowLen) { return rowLen | 1; }
// Rows per LDS chunk: as many as fit kPackLdsBytes, at most 64 and a
// multiple of 4 (a chunk's first row then starts 16-byte aligned in the
// output whenever the row length is even), at least 8.
HDI int packChunkRows(int rowLen)
{
    const int fit = kPackLdsBytes / (packStride(rowLen) * 4);
    const int rows = (fit < 64 ? fit : 64) & ~3;
    return rows > 8 ? rows : 8;
}
HDI size_t packLdsBytes(int rowLen) { return (size_t)packChunkRows(rowLen) * packStride(rowLen) * sizeof(float); }

typedef float F4v __attribute__((ext_vector_type(4)));

// A workgroup barrier that orders LDS accesses only: every thread's LDS reads
// and writes before it complete before any thread's after it, while its
// global stores may still be in flight (__syncthreads waits for those too).
// The packing rounds store a chunk's rows from LDS and then rebuild the LDS
// with the next chunk: nothing in the workgroup reads the stored rows, so the
// stores' latency need not be waited for before the rebuild.
DI void ldsBarrier()
{
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
    __builtin_amdgcn_s_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}

// Stores `rows` whole rows (rowLen floats each, row stride `stride` floats in
// LDS from `lds`) to the contiguous run at dst; 16 bytes per lane and
// instruction when dst is 16-byte aligned.  The stores are non-temporal: the
// rows are not read again by the step, and streaming them past the caches
// keeps the state words the later stages re-read cached (packing 36.6 ->
// 34.3 us).  Called by every thread of the workgroup.
DI void storeRunFromLds(float* dst, int rowLen, int stride, int rows, const float* lds)
{
    const int t = threadIdx.x, total = rows * rowLen;
    if (((size_t)dst & 15) == 0) {
        const int step = 4 * kPackBlock, rs = step / rowLen, cs = step % rowLen;
        int rr = 4 * t / rowLen, c = 4 * t % rowLen;
        for (int e = 4 * t; e + 3 < total; e += step) {
            float v[4];
            int r2 = rr, c2 = c;
#pragma unroll
            for (int k = 0; k < 4; k++) {
                v[k] = lds[r2 * stride + c2];
                if (++c2 == rowLen) { c2 = 0; r2++; }
            }
            const F4v run = { v[0], v[1], v[2], v[3] };
            __builtin_nontemporal_store(run, reinterpret_cast<F4v*>(dst + e));
            rr += rs;
            c += cs;
            if (c >= rowLen) { c -= rowLen; rr++; }
        }
        const int e = (total & ~3) + t;
        if (e < total) __builtin_nontemporal_store(lds[(e / rowLen) * stride + e % rowLen], dst + e);
        return;
    }
    const int rowStep = kPackBlock / rowLen, colStep = kPackBlock % rowLen;
    int rr = t / rowLen, c = t % rowLen;
    for (int e = t; e < total; e += kPackBlock) {
        __builtin_nontemporal_store(lds[rr * stride + c], dst + e);
        rr += rowStep;
        c += colStep;
        if (c >= rowLen) { c -= rowLen; rr++; }
    }
}

// Rows [r0, r1) of out (rowLen floats each): a row r with keep(r) is built by
// part(r, q, dst) for q = 0..kRowParts-1 and stored; other rows are left
// untouched.  Every thread of the workgroup calls this (it holds barriers);
// on return every part() call of the workgroup has completed.
template <typename Keep, typename Part>
DI void packRowsParts(float* out, int rowLen, int r0, int r1, Keep&& keep, Part&& part)
{
    extern __shared__ float packLds[];
    __shared__ int on[64];
    const int t = threadIdx.x, lane = t & 63, q = t >> 6;
    const int stride = packStride(rowLen), chunk = packChunkRows(rowLen);
    const int rowStep = kPackBlock / rowLen, colStep = kPackBlock % rowLen;
    for (int c0 = r0; c0 < r1; c0 += chunk) {
        const int rows = min(chunk, r1 - c0);
        // keep() depends on the row only: every wave sees the same rows
        const bool mine = lane < rows && keep(c0 + lane);
        const int kept = __popcll(__ballot(mine));
        if (kept == 0) continue;
        if (q == 0) on[lane] = mine;
        if (mine) part(c0 + lane, q, packLds + lane * stride);
        ldsBarrier();
        float* dst = out + (size_t)c0 * rowLen;
        if (kept == rows) {
            // every row kept: the chunk is one contiguous run
            storeRunFromLds(dst, rowLen, stride, rows, packLds);
        } else {
            const int total = rows * rowLen;
            int rr = t / rowLen, c = t % rowLen;
            for (int e = t; e < total; e += kPackBlock) {
                if (on[rr]) dst[e] = packLds[rr * stride + c];
                rr += rowStep;
                c += colStep;
                if (c >= rowLen) { c -= rowLen; rr++; }
            }
        }
        ldsBarrier();
    }
}

__global__ __launch_bounds__(kPackBlock) void stateKernel(Dev d, float* out, int stateDimV, int touchWindow,
                                                         int tickCount, const bool* mask)
{
    const int r0 = blockIdx.x * packChunkRows(stateDimV);
    packRowsParts(
        out, stateDimV, r0, min(r0 + packChunkRows(stateDimV), d.nSim), [&](int s) { return !mask || mask[s]; },
        [&](int s, int q, float* o) { packStatePart(d, s, touchWindow, tickCount, q, o); });
}

__global__ __launch_bounds__(kPackBlock) void obsKernel(Dev d, float* out, int obsDimV, const bool* mask, int invert,
                                                       int normalizeObs, int prev)
{
    const int r0 = blockIdx.x * packChunkRows(obsDimV);
    packRowsParts(
        out, obsDimV, r0, min(r0 + packChunkRows(obsDimV), d.nTotal),
        [&](int a) { return !mask || mask[a / d.nCars]; },
        [&](int a, int q, float* o) {
            packObservationPart(d, a / d.nCars, a % d.nCars, invert != 0, normalizeObs != 0, prev != 0, q, o);
        });
}

// Rows rowOf(i), i in [i0, i1), of out (rowLen floats each), built by
// part(row, q, dst) for q = 0..kRowParts-1 as packRowsParts builds them, and
// each stored as its own contiguous run (the rows of a compacted selection
// are scattered through out).  Every thread of the workgroup calls this.
template <typename RowOf, typename Part>
DI void packRowsGathered(float* out, int rowLen, int i0, int i1, RowOf&& rowOf, Part&& part)
{
    extern __shared__ float packLds[];
    __shared__ int rowAt[64];
    const int t = threadIdx.x, lane = t & 63, q = t >> 6;
    const int stride = packStride(rowLen), chunk = packChunkRows(rowLen);
    const int rowStep = kPackBlock / rowLen, colStep = kPackBlock % rowLen;
    for (int c0 = i0; c0 < i1; c0 += chunk) {
        const int rows = min(chunk, i1 - c0);
        const int row = lane < rows ? rowOf(c0 + lane) : 0;
        if (q == 0) rowAt[lane] = row;
        if (lane < rows) part(row, q, packLds + lane * stride);
        ldsBarrier();
        const int total = rows * rowLen;
        int rr = t / rowLen, c = t % rowLen;
        for (int e = t; e < total; e += kPackBlock) {
            __builtin_nontemporal_store(packLds[rr * stride + c], out + (size_t)rowAt[rr] * rowLen + c);
            rr += rowStep;
            c += colStep;
            if (c >= rowLen) { c -= rowLen; rr++; }
        }
        ldsBarrier();
    }
}

// The state rows of the simulations list[0..*count).
__global__ __launch_bounds__(kPackBlock) void stateListKernel(Dev d, float* out, int stateDimV, int touchWindow,
                                                             int tickCount, const int* list, const int* count)
{
    const int i0 = blockIdx.x * packChunkRows(stateDimV), n = *count;
    if (i0 >= n) return;
    packRowsGathered(
        out, stateDimV, i0, min(i0 + packChunkRows(stateDimV), n), [&](int i) { return list[i]; },
        [&](int s, int q, float* o) { packStatePart(d, s, touchWindow, tickCount, q, o); });
}

// The observation rows of the cars of the simulations list[0..*count).
__global__ __launch_bounds__(kPackBlock) void obsListKernel(Dev d, float* out, int obsDimV, int invert,
                                                           int normalizeObs, int prev, const int* list,
                                                           const int* count)
{
    const int i0 = blockIdx.x * packChunkRows(obsDimV), n = *count * d.nCars;
    if (i0 >= n) return;
    packRowsGathered(
        out, obsDimV, i0, min(i0 + packChunkRows(obsDimV), n),
        [&](int i) { return list[i / d.nCars] * d.nCars + i % d.nCars; },
        [&](int a, int q, float* o) {
            packObservationPart(d, a / d.nCars, a % d.nCars, invert != 0, normalizeObs != 0, prev != 0, q, o);
        });
}

// Everything an env step does after its ticks, for kStepSims simulations per
// workgroup: rewards and dones, the transition state and the transition
// observations of finished simulations, their resets, the match state, the
// observations and the state, with the reference's data dependences (the
// transition rows read the state before the resets, the others after).  A
// simulation's rows depend on nothing but its own state, so the workgroup
// needs only its own barriers.  Every wave decides the fate of the
// workgroup's simulations (one per lane) from their match words, so the
// finished ones are known to each wave without a barrier; the transition
// observations of the first finished ones are built in the same round as
// the transition state, in the LDS left over by the state rows.
constexpr int kStepSims = 64;
static_assert(kStepSims == 64, "one simulation per lane of each wave");

struct StepIO {
    float *rewards, *tstate, *tobs, *obs, *state;
    bool *dones, *tovertime, *overtime;
    int32_t *tscore, *tticks, *score, *ticks;
    const uint32_t* actions;  // the step's actions, 7 words per car ...
    uint32_t* actionCopy;     // ... kept here (null: not kept)
    int obsDim, stateDim, invert, normalize, prev, frameskip, tickCount, nOrange;
    DoneRule rule;
};

HDI size_t stepLdsBytes(int obsDim, int stateDim)
{
    const size_t a = packLdsBytes(obsDim), b = packLdsBytes(stateDim);
    return a > b ? a : b;
}

__global__ __launch_bounds__(kPackBlock) void stepEnvKernel(Dev d, StepIO io)
{
    extern __shared__ float packLds[];
    __shared__ int listedRow[64];   // tobs row of each transition observation built in round 1
    const int t = threadIdx.x, lane = t & 63, q = t >> 6, nC = d.nCars;
    const int s0 = blockIdx.x * kStepSims, s1 = min(s0 + kStepSims, d.nSim);
    const int s = s0 + lane;
    // the match words and the first action words are loaded first and used
    // after the transition state's loads have been issued
    MatchWords m{};
    if (s < s1) m = matchWords(d, s);
    constexpr int kCopyRegs = 4;   // action words per thread held in registers (all of them in 1v1)
    const int copyWords = io.actionCopy ? (s1 - s0) * nC * 7 : 0;
    const size_t w0 = (size_t)s0 * nC * 7;
    uint32_t act[kCopyRegs];
#pragma unroll
    for (int i = 0; i < kCopyRegs; i++) act[i] = t + i * kPackBlock < copyWords ? io.actions[w0 + t + i * kPackBlock] : 0u;

    // round 1: the first chunk of transition state rows, and as many
    // transition observation rows as fit beside them
    const int sStride = packStride(io.stateDim), oStride = packStride(io.obsDim);
    // when the state rows take several chunks, the first one is an even
    // share (a multiple of 4), which leaves LDS for more transition
    // observations beside it
    const int sChunk = packChunkRows(io.stateDim), sChunks = (s1 - s0 + sChunk - 1) / sChunk;
    const int aRows = min((((s1 - s0 + sChunks - 1) / sChunks) + 3) & ~3, min(sChunk, s1 - s0));
    if (lane < aRows) packStatePart(d, s0 + lane, io.frameskip, io.tickCount, q, packLds + lane * sStride);

    int outcome = kKept;
    bool dn = false;
    if (s < s1) {
        dn = simDoneFrom(m, io.tickCount, io.rule);
        outcome = doneOutcome(m, io.tickCount, io.rule);
        if (q == 0) {
            io.rewards[s] = (float)m.scorer;
            io.dones[s] = dn;
            io.tscore[s] = m.blue - m.orange;
            io.tticks[s] = m.ep;
            io.tovertime[s] = m.overtime != 0;
            io.score[s] = outcome == kReset ? 0 : m.blue - m.orange;
            io.ticks[s] = outcome == kReset ? 0 : m.ep;
            io.overtime[s] = outcome == kReset ? false : (outcome == kOvertimeEntered || m.overtime != 0);
        }
    }
    // the finished simulations, the same mask in every wave; the transition
    // observation rows of finished simulation j (in lane order) are
    // doneRank(j) * nC .. + nC - 1
    const uint64_t doneMask = __ballot(dn);
    const int doneRows = __popcll(doneMask) * nC;
    auto doneRank = [&](int local) { return __popcll(doneMask & ((1ull << local) - 1ull)); };
    float* const ldsB = packLds + aRows * sStride;
    const int capB = ((int)(stepLdsBytes(io.obsDim, io.stateDim) / sizeof(float)) - aRows * sStride) / oStride;
    const int nB = min(doneRows, min(max(capB, 0), 64));   // listedRow holds 64
    if (lane < nB) {
        // the lane-th finished row: its simulation is the (lane / nC)-th set bit of doneMask
        uint64_t m = doneMask;
        for (int k = 0; k < lane / nC; k++) m &= m - 1ull;
        const int local = __ffsll((unsigned long long)m) - 1;
        packObservationPart(d, s0 + local, lane % nC, io.invert != 0, io.normalize != 0, io.prev != 0, q,
                            ldsB + lane * oStride);
        if (q == 0) listedRow[lane] = (s0 + local) * nC + lane % nC;
    }
    ldsBarrier();
    storeRunFromLds(io.tstate + (size_t)s0 * io.stateDim, io.stateDim, sStride, aRows, packLds);
    {
        // the listed rows, each a contiguous run of obsDim floats in tobs
        const int total = nB * io.obsDim;
        for (int e = t; e < total; e += kPackBlock) {
            const int j = e / io.obsDim, c = e % io.obsDim;
            __builtin_nontemporal_store(ldsB[j * oStride + c], io.tobs + (size_t)listedRow[j] * io.obsDim + c);
        }
    }
    ldsBarrier();
    // the rest of the transition state (more cars than one chunk holds) and
    // the transition observations that did not fit
    if (s0 + aRows < s1)
        packRowsParts(
            io.tstate, io.stateDim, s0 + aRows, s1, [](int) { return true; },
            [&](int r, int qq, float* o) { packStatePart(d, r, io.frameskip, io.tickCount, qq, o); });
    if (doneRows > nB)
        packRowsParts(
            io.tobs, io.obsDim, s0 * nC, s1 * nC,
            [&](int a) {
                const int local = a / nC - s0;
                return ((doneMask >> local) & 1ull) != 0 && doneRank(local) * nC + a % nC >= nB;
            },
            [&](int a, int qq, float* o) {
                packObservationPart(d, a / nC, a % nC, io.invert != 0, io.normalize != 0, io.prev != 0, qq, o);
            });
    if (s < s1) applyDoneOutcomePart(d, s, outcome, io.tickCount, io.nOrange, q);
    __syncthreads();
    packRowsParts(
        io.obs, io.obsDim, s0 * nC, s1 * nC, [](int) { return true; },
        [&](int a, int qq, float* o) {
            packObservationPart(d, a / nC, a % nC, io.invert != 0, io.normalize != 0, io.prev != 0, qq, o);
        });
    packRowsParts(
        io.state, io.stateDim, s0, s1, [](int) { return true; },
        [&](int r, int qq, float* o) { packStatePart(d, r, 1, io.tickCount, qq, o); });
    // the kept copy of the step's actions
#pragma unroll
    for (int i = 0; i < kCopyRegs; i++)
        if (t + i * kPackBlock < copyWords) io.actionCopy[w0 + t + i * kPackBlock] = act[i];
    for (int w = t + kCopyRegs * kPackBlock; w < copyWords; w += kPackBlock) io.actionCopy[w0 + w] = io.actions[w0 + w];
}

// The rows a mask sets, compacted into list[0..*count): each thread scans
// kCompactRows consecutive rows, a workgroup scan places the threads' rows,
// and each workgroup takes its place in the list with one atomic add on the
// count (which clearCountKernel zeroes first).  The workgroups' order in the
// list varies from run to run; nothing depends on it, as every row's reset
// and repacking touch that row's simulation only.
__global__ void clearCountKernel(int* count) { *count = 0; }

constexpr int kCompactBlock = 256;
constexpr int kCompactRows = 16;
__global__ __launch_bounds__(kCompactBlock) void compactMaskKernel(const uint8_t* __restrict__ mask, int n,
                                                                   int* __restrict__ list, int* __restrict__ count)
{
    __shared__ int waveBase[kCompactBlock / 64 + 1];
    const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
    const int r0 = (blockIdx.x * kCompactBlock + t) * kCompactRows;
    unsigned bits = 0;
#pragma unroll
    for (int k = 0; k < kCompactRows; k++)
        if (r0 + k < n && mask[r0 + k] != 0) bits |= 1u << k;
    const int c = __popc(bits);
    const int incl = waveInclusiveScan(c);
    if (lane == 63) waveBase[wave] = incl;
    __syncthreads();
    if (t == 0) {
        int total = 0;
        for (int w = 0; w < kCompactBlock / 64; w++) {
            const int v = waveBase[w];
            waveBase[w] = total;
            total += v;
        }
        waveBase[kCompactBlock / 64] = total ? atomicAdd(count, total) : 0;
    }
    __syncthreads();
    int at = waveBase[kCompactBlock / 64] + waveBase[wave] + incl - c;
#pragma unroll
    for (int k = 0; k < kCompactRows; k++)
        if (bits & (1u << k)) list[at++] = r0 + k;
}

__global__ void setBallKernel(Dev d, const float* pos, const float* vel, const float* ang, Selection sel)
{
    const int r = selectedInput(sel, blockIdx.x * blockDim.x + threadIdx.x);
    if (r < 0) return;
    const int t = selectRow(sel, r, d.nSim);
    if (t < 0) return;
    d.ssetv(CARL_SIM_BALL_POS, t, V3{ pos[3 * r], pos[3 * r + 1], pos[3 * r + 2] });
    d.ssetv(CARL_SIM_BALL_VEL, t, V3{ vel[3 * r], vel[3 * r + 1], vel[3 * r + 2] });
    d.ssetv(CARL_SIM_BALL_ANG, t, V3{ ang[3 * r], ang[3 * r + 1], ang[3 * r + 2] });
    d.ssetv(CARL_SIM_BALL_IMP, t, kZero);
}

__global__ void setCarKernel(Dev d, const float* pos, const float* rot, const float* vel, const float* ang,
                             const void* demoed, int byteDemoed, const float* boost, const float* internal,
                             Selection sel)
{
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    const int r = selectedInput(sel, i / d.nCars);
    if (r < 0) return;
    const int t = selectRow(sel, r, d.nSim);
    if (t < 0) return;
    const int local = i % d.nCars;
    setCarRow(d, r * d.nCars + local, t, local, pos, rot, vel, ang, demoed, byteDemoed != 0, boost, internal);
}

// Wheel contacts of the selected cars against the restored scene (rays only,
// searched cooperatively like the contact kernel).  One wave per block.
__global__ __launch_bounds__(kContactBlock) void refreshKernel(Dev d, Selection sel, int screen)
{
    __shared__ ContactLds L;
    const int lane = threadIdx.x;
    // a compacted selection's blocks past its cars have nothing to do
    if (sel.list && blockIdx.x * kContactOwners >= *sel.count * d.nCars) return;
    const int i = blockIdx.x * kContactOwners + lane;
    int car = -1;
    if (lane < kContactOwners) {
        const int r = selectedInput(sel, i / d.nCars);
        const int t = r < 0 ? -1 : selectRow(sel, r, d.nSim);
        if (t >= 0) car = t * d.nCars + i % d.nCars;
    }
    const bool active = car >= 0 && !d.ci(CARL_CAR_DEMOED, car);
    V3 cen = kZero;
    Q4 rot{ 0.f, 0.f, 0.f, 1.f };
    Broad bp{ 0, 0, 0 };
    if (active) {
        cen = d.cv(CARL_CAR_CEN, car);
        rot = d.cq(CARL_CAR_ROT, car);
        bp = broadphase(d, d.cv(CARL_CAR_POS, car), d.cv(CARL_CAR_VEL, car), d.cv(CARL_CAR_ANG, car), cen, rot);
    }
    contactPrepare(L, lane, false, cen, rot, bp.start, false, bp.cell, screen != 0);
    __syncthreads();
    waveItemsPipelined(
        bp.count, L.excl, [&](int o, int q, bool valid) { return contactFetch(d, L, o, q, valid); },
        [&](const RefBox& b, int o, int, int) { contactScreen(L, b, o, lane); },
        [&](bool last) { contactDrain(d, L, lane, last); });
    __syncthreads();
    if (car < 0) return;
    if (!active) {
        clearWheelContacts(d, car);
        return;
    }
    Wheels w;
    (void)contactFinish(d, L, lane, car, car / d.nCars, cen, rot, w);
    storeRefreshedWheels(d, car, w);
}

__global__ void setMatchKernel(Dev d, const int32_t* blue, const int32_t* orange, const int32_t* ticks, Selection sel)
{
    const int r = selectedInput(sel, blockIdx.x * blockDim.x + threadIdx.x);
    if (r < 0) return;
    const int t = selectRow(sel, r, d.nSim);
    if (t < 0) return;
    d.sseti(CARL_SIM_BLUE_SCORE, t, blue[r]);
    d.sseti(CARL_SIM_ORANGE_SCORE, t, orange[r]);
    d.sseti(CARL_SIM_LAST_SCORER, t, 0);
    d.sseti(CARL_SIM_OVERTIME, t, 0);
    d.sseti(CARL_SIM_EPISODE_TICKS, t, ticks[r]);
}

__global__ void resetPadsKernel(Dev d, Selection sel)
{
    const int r = selectedInput(sel, blockIdx.x * blockDim.x + threadIdx.x);
    if (r < 0) return;
    const int t = selectRow(sel, r, d.nSim);
    if (t < 0) return;
    for (int p = 0; p < kPads; p++) d.ssetf(CARL_SIM_PAD_COOLDOWN + p, t, 0.f);
}

// ---- exclusive scan (no library): per-tile wave64 DPP scans, tile totals
// scanned recursively and added back.
constexpr int kScanBlock = 256;
constexpr int kScanItems = 8;
constexpr int kScanTile = kScanBlock * kScanItems;

// exclusive scan of one tile per block; block totals to `sums` when given
__global__ __launch_bounds__(kScanBlock) void scanTileKernel(const int32_t* in, int32_t* out, int n, int32_t* sums)
{
    __shared__ int waveTotals[kScanBlock / 64];
    const int base = blockIdx.x * kScanTile + threadIdx.x * kScanItems;
    int v[kScanItems];
    int local = 0;
#pragma unroll
    for (int i = 0; i < kScanItems; i++) {
        v[i] = base + i < n ? in[base + i] : 0;
        local += v[i];
    }
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int incl = waveInclusiveScan(local);
    if (lane == 63) waveTotals[wave] = incl;
    __syncthreads();
    int waveOffset = 0;
    for (int w = 0; w < wave; w++) waveOffset += waveTotals[w];
    int run = waveOffset + incl - local;
#pragma unroll
    for (int i = 0; i < kScanItems; i++) {
        if (base + i < n) out[base + i] = run;
        run += v[i];
    }
    if (sums && threadIdx.x == kScanBlock - 1) sums[blockIdx.x] = waveOffset + incl;
}

__global__ void scanAddKernel(int32_t* out, int n, const int32_t* offsets)
{
    const int i = blockIdx.x * kScanTile + threadIdx.x;
    for (int k = 0; k < kScanItems; k++) {
        const int idx = i + k * kScanBlock;
        if (idx < n) out[idx] += offsets[blockIdx.x];
    }
}

// 32-bit words of tile sums and their scan that runScanInto needs for n items
// (every level of the recursion; 0 when one tile holds them all).
size_t scanWorkWords(int n)
{
    const int tiles = (n + kScanTile - 1) / kScanTile;
    return tiles <= 1 ? 0 : 2 * (size_t)tiles + scanWorkWords(tiles);
}

// Scan with the tile sums of every level in `work` (scanWorkWords(n) words
// of device memory); every word of it is written before it is read.
int runScanInto(const int32_t* in, int32_t* out, int n, hipStream_t stream, int32_t* work)
{
    if (n <= 0) return CARL_OK;
    const int tiles = (n + kScanTile - 1) / kScanTile;
    if (tiles == 1) {
        scanTileKernel<<<1, kScanBlock, 0, stream>>>(in, out, n, nullptr);
        HIP_TRY(hipGetLastError());
        return CARL_OK;
    }
    int32_t* sums = work;
    int32_t* offsets = work + tiles;
    scanTileKernel<<<tiles, kScanBlock, 0, stream>>>(in, out, n, sums);
    HIP_TRY(hipGetLastError());
    const int rc = runScanInto(sums, offsets, tiles, stream, work + 2 * (size_t)tiles);
    if (rc != CARL_OK) return rc;
    scanAddKernel<<<tiles, kScanBlock, 0, stream>>>(out, n, offsets);
    HIP_TRY(hipGetLastError());
    return CARL_OK;
}

int runScan(const int32_t* in, int32_t* out, int n, hipStream_t stream)
{
    const size_t words = scanWorkWords(n);
    if (words == 0) return runScanInto(in, out, n, stream, nullptr);
    int32_t* work = nullptr;
    HIP_TRY(hipMallocAsync((void**)&work, sizeof(int32_t) * words, stream));
    const int rc = runScanInto(in, out, n, stream, work);
    const hipError_t freed = hipFreeAsync(work, stream);
    if (rc != CARL_OK) return rc;
    HIP_TRY(freed);
    return CARL_OK;
}

// ---- the scan's tile sums in a fixed device array, for callers that cannot
// allocate.  One copy per GPU; every call on a GPU shares it.
constexpr int kScanNoAllocMaxItems = 1 << 26;
constexpr size_t kScanScratchWords = 2 * (kScanNoAllocMaxItems / kScanTile) + 2 * 16;
static_assert(kScanNoAllocMaxItems % kScanTile == 0, "whole tiles at the maximum");
static_assert((kScanNoAllocMaxItems / kScanTile) <= 16 * kScanTile, "two sum levels cover the maximum");

static __device__ __align__(256) int32_t scratch[kScanScratchWords];

constexpr int kMaxDevices = 64;
std::mutex scratchMutex;
int32_t* scratchAddress[kMaxDevices] = {};

// Device address of `scratch` on the current device, looked up once per
// device (the host-side name is not a device address).
int scratchOnCurrentDevice(int32_t** out)
{
    int device = 0;
    HIP_TRY(hipGetDevice(&device));
    if (device < 0 || device >= kMaxDevices) return fail(CARL_ERR_RUNTIME, "device ordinal out of range");
    std::lock_guard<std::mutex> lock(scratchMutex);
    if (!scratchAddress[device]) {
        void* ptr = nullptr;
        HIP_TRY(hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch)));
        if (!ptr) return fail(CARL_ERR_RUNTIME, "scan scratch has no device address");
        scratchAddress[device] = (int32_t*)ptr;
    }
    *out = scratchAddress[device];
    return CARL_OK;
}

std::string libraryDir()
{
    Dl_info info{};
    if (dladdr((void*)&libraryDir, &info) && info.dli_fname) {
        std::string p = info.dli_fname;
        const size_t slash = p.rfind('/');
        if (slash != std::string::npos) return p.substr(0, slash);
    }
    return ".";
}

// ------------------------------------------------------------ shared arena

// The arena is read-only, so the environments on one device share a single
// device copy of it, refcounted and freed with the last of them.  The host
// build is made once per process for each mesh file and metadata file (the
// reference builds its host mesh once per process in static locals,
// src/ArenaMesh.cu:17-28, and gives every environment a device copy).  A
// file is identified by its path, size and modification time, so a file
// rewritten in place is built again.
struct DeviceArena {
    std::string key;
    int device = 0;
    int refs = 0;
    std::vector<void*> blocks;   // the device allocations, freed together
    ArenaView view{};
};

std::mutex arenaMutex;
std::vector<std::pair<std::string, std::shared_ptr<const HostArena>>> hostArenas;
std::vector<DeviceArena*> deviceArenas;

std::string fileKey(const std::string& path)
{
    struct stat st {};
    if (stat(path.c_str(), &st) != 0) return path + "|absent";
    return path + "|" + std::to_string((long long)st.st_size) + "|" + std::to_string((long long)st.st_mtim.tv_sec)
           + "." + std::to_string((long long)st.st_mtim.tv_nsec);
}

// The host build for `key`, made on first use; a failed build is not kept.
// Called with arenaMutex held.
int hostArenaFor(const std::string& key, const std::string& obj, const char* meta,
                 std::shared_ptr<const HostArena>* out)
{
    for (const auto& kv : hostArenas)
        if (kv.first == key) {
            *out = kv.second;
            return CARL_OK;
        }
    auto host = std::make_shared<HostArena>();
    std::string err = buildArena(obj, *host);
    // the native mesh metadata, when named (src/ArenaMesh.cu:69-99)
    if (err.empty() && meta) err = readArenaMetadata(meta, *host);
    if (!err.empty()) return fail(CARL_ERR_ARENA, err);
    hostArenas.emplace_back(key, host);
    *out = host;
    return CARL_OK;
}

template <typename T, typename S>
int uploadBlock(DeviceArena* a, const S* src, size_t bytes, const T** dst)
{
    void* p = nullptr;
    HIP_TRY(hipMalloc(&p, std::max<size_t>(bytes, 16)));
    a->blocks.push_back(p);
    if (bytes) HIP_TRY(hipMemcpy(p, src, bytes, hipMemcpyHostToDevice));
    *dst = (const T*)p;
    return CARL_OK;
}

void freeDeviceArena(DeviceArena* a)
{
    for (void* p : a->blocks) (void)hipFree(p);
    delete a;
}

int uploadArena(const HostArena& host, DeviceArena* a)
{
    ArenaView& v = a->view;
    std::vector<float4> ang(host.angles.size() / 3);
    for (size_t t = 0; t < ang.size(); t++)
        ang[t] = make_float4(host.angles[3 * t], host.angles[3 * t + 1], host.angles[3 * t + 2], 0.f);
    auto bytes = [](const auto& vec) { return vec.size() * sizeof(vec[0]); };
    CARL_TRY(uploadBlock(a, host.records.data(), bytes(host.records), &v.rec));
    CARL_TRY(uploadBlock(a, host.cellStart.data(), bytes(host.cellStart), &v.cellStart));
    CARL_TRY(uploadBlock(a, ang.data(), bytes(ang), &v.angles));
    CARL_TRY(uploadBlock(a, host.triRecords.data(), bytes(host.triRecords), &v.tri));
    CARL_TRY(uploadBlock(a, host.cellTris.data(), bytes(host.cellTris), &v.cellTri));
    CARL_TRY(uploadBlock(a, host.triBoxes.data(), bytes(host.triBoxes), &v.triBox));
    CARL_TRY(uploadBlock(a, host.triAux.data(), bytes(host.triAux), &v.triAux));
    CARL_TRY(uploadBlock(a, host.fineRecords.data(), bytes(host.fineRecords), &v.fineRec));
    CARL_TRY(uploadBlock(a, host.fineAux.data(), bytes(host.fineAux), &v.fineAux));
    CARL_TRY(uploadBlock(a, host.carStart.data(), bytes(host.carStart), &v.carStart));
    CARL_TRY(uploadBlock(a, host.carTris.data(), bytes(host.carTris), &v.carTri));
    CARL_TRY(uploadBlock(a, host.fineStart.data(), bytes(host.fineStart), &v.fineStart));
    v.native = nullptr;
    if (!host.nativeRecords.empty())
        CARL_TRY(uploadBlock(a, host.nativeRecords.data(), bytes(host.nativeRecords), &v.native));
    return CARL_OK;
}

// The arena named by CARL_ARENA_OBJ (else the packaged mesh) and
// CARL_ARENA_METADATA on the current device, one more reference to it.  The
// host build and its errors come before any device work.
int acquireArena(DeviceArena** out)
{
    *out = nullptr;
    const std::string obj = findArenaObj(libraryDir());
    const char* meta = std::getenv("CARL_ARENA_METADATA");
    const std::string key = fileKey(obj) + "\n" + (meta ? fileKey(meta) : std::string("-"));
    std::lock_guard<std::mutex> lock(arenaMutex);
    std::shared_ptr<const HostArena> host;
    CARL_TRY(hostArenaFor(key, obj, meta, &host));
    int device = 0;
    HIP_TRY(hipGetDevice(&device));
    for (DeviceArena* a : deviceArenas)
        if (a->device == device && a->key == key) {
            a->refs++;
            *out = a;
            return CARL_OK;
        }
    auto* a = new DeviceArena();
    a->key = key;
    a->device = device;
    const int rc = uploadArena(*host, a);
    if (rc) {
        freeDeviceArena(a);
        return rc == CARL_ERR_RUNTIME ? fail(CARL_ERR_RUNTIME, "arena upload failed: " + g_lastError) : rc;
    }
    a->refs = 1;
    deviceArenas.push_back(a);
    *out = a;
    return CARL_OK;
}

void releaseArena(DeviceArena* a)
{
    if (!a) return;
    std::lock_guard<std::mutex> lock(arenaMutex);
    if (--a->refs > 0) return;
    deviceArenas.erase(std::find(deviceArenas.begin(), deviceArenas.end(), a));
    freeDeviceArena(a);
}

// The tiled state blocks and the tick workspace are addressed through 32-bit
// buffer resources (a byte count and a 32-bit byte offset per access), so
// each must stay below 2^31 bytes: at most kMaxCars cars in all (the car
// block, 4 * CARL_CAR_FIELDS bytes per car, is the largest of the three).
constexpr long long kMaxCars = (INT_MAX / (4LL * CARL_CAR_FIELDS)) & ~63LL;
static_assert(kMaxCars * 4LL * kWsPlanes <= INT_MAX && kMaxCars * 4LL * CARL_SIM_FIELDS <= INT_MAX,
              "the car block bounds the workspace and the simulation block");

int checkSizes(int nSim, int nCars)
{
    const long long cars = (long long)nSim * nCars;
    if (cars > kMaxCars)
        return fail(CARL_ERR_VALUE, "n_sim * cars per simulation must be at most " + std::to_string(kMaxCars)
                                        + " (the state's 32-bit byte offsets); got " + std::to_string(cars));
    return CARL_OK;
}

}  // namespace

// ------------------------------------------------------------------- engine

struct carl_env {
    int nSim = 0, nBlue = 0, nOrange = 0, nCars = 0, nTotal = 0, seed = 0;
    int frameskip = 1;
    bool invert = true, normalize = false, prevControls = false;
    int obsDim = 0, stateDim = 0;
    int maxTicks = kRegulationTicks, overtimeTicks = kRegulationTicks, noTouchTicks = 0;
    int tickCount = 0;
    hipStream_t stream = nullptr;
    uint32_t* car = nullptr;
    uint32_t* sim = nullptr;
    DeviceArena* arena = nullptr;        // shared with the other environments on the device
    float *obs = nullptr, *tobs = nullptr, *state = nullptr, *tstate = nullptr, *rewards = nullptr;
    bool *dones = nullptr, *overtime = nullptr, *tovertime = nullptr;
    int32_t *score = nullptr, *ticks = nullptr, *tscore = nullptr, *tticks = nullptr;
    int32_t* actions = nullptr;
    float* cactions = nullptr;
    uint32_t* ws = nullptr;  // per-tick car workspace (kWsPlanes planes)
    int* rowList = nullptr;  // a masked reset's selected rows (n_sim), then their count
    // 1v1: the deal of balanced window launches, kDealSets sets of class
    // counts and lists, and the balanced launches so far
    int* dealCount = nullptr;
    int* dealList = nullptr;
    long long dealLaunches = 0;
    int balance = 1;                     // deal 1v1 window launches by cost
    float* ballScratch = nullptr;    // with it: kNativeMaxContacts slots of kNativeSlotWords per simulation
    int tickStreams = 1;                 // partitions of the tick, one stream each
    int contactScreen = 1;               // screen (car, triangle) pairs in the contact search
    hipStream_t aux[kMaxTickStreams - 1] = {};
    hipEvent_t fork = nullptr, join[kMaxTickStreams - 1] = {};
    int windowSims = kDefaultWindowSims;  // simulations per block of the tick-window kernel (0: phase kernels)
    // Until the caller sets windowSims, a run too small to fill the device's
    // resident window workgroups uses smaller ones (down to kAutoWindowMin
    // simulations): the kernel's time is one workgroup's latency chain, so
    // spreading the simulations over more compute units shortens it.
    bool windowAuto = true;
    int windowResident = 0;   // window workgroups the device holds at once
    int timing = 0;                      // CARL_TIME_* flags
    // timing: a start and an end event per timed launch not yet folded
    // (a pool of at most kTimedPool pairs) and the launch's kernel id;
    // folding adds their durations to the sums below
    size_t timedLaunches = 0;
    std::vector<hipEvent_t> marks;
    std::vector<int> markKernel;
    double kernelMs[CARL_TICK_KERNELS] = {};
    int kernelLaunches[CARL_TICK_KERNELS] = {};
    // stage profile (CARL_TIME_STAGES): the window kernel's clock counters
    // (kProfWords), the launch durations of the profiled ticks, their count,
    // and the workgroups one profiled launch keeps resident together
    unsigned long long* prof = nullptr;
    double stageKernelMs[CARL_TICK_KERNELS] = {};
    int stageTicks = 0;
    int stagePath = 0;  // 1: window kernel, 2: phase kernels
    int profResident = 0;  // window workgroups the device holds at once
    int profSlots = 0;     // of those, the ones a profiled launch fills
    bool profMixed = false;  // profiled launches of different shapes
    double clockMHz = 0.0;  // the wall clock read by wall_clock64

    Dev dev() const
    {
        Dev d;
        d.car = car; d.sim = sim; d.nSim = nSim; d.nBlue = nBlue; d.nCars = nCars; d.nTotal = nTotal; d.seed = seed;
        d.arena = arena->view;
        d.ballScratch = ballScratch;
        return d;
    }
    DoneRule rule() const { return DoneRule{ maxTicks, overtimeTicks, noTouchTicks }; }
    // native mesh metadata (CARL_ARENA_METADATA)
    bool native() const { return arena && arena->view.native; }
    int grid(int n, int block) const { return (n + block - 1) / block; }
};

namespace {

template <typename T>
int devAlloc(T** p, size_t count)
{
    HIP_TRY(hipMalloc((void**)p, std::max<size_t>(count, 1) * sizeof(T)));
    HIP_TRY(hipMemset(*p, 0, std::max<size_t>(count, 1) * sizeof(T)));
    return CARL_OK;
}

void freeAll(carl_env* e)
{
    void* ptrs[] = { e->car, e->sim, e->obs, e->tobs, e->state, e->tstate, e->rewards, e->dones,
                     e->overtime, e->tovertime, e->score, e->ticks, e->tscore, e->tticks, e->actions, e->cactions,
                     e->ws, e->prof, e->ballScratch, e->rowList, e->dealCount, e->dealList };
    for (void* p : ptrs)
        if (p) (void)hipFree(p);
    releaseArena(e->arena);
    e->arena = nullptr;
    for (hipEvent_t ev : e->marks) (void)hipEventDestroy(ev);
    for (int i = 0; i < kMaxTickStreams - 1; i++) {
        if (e->join[i]) (void)hipEventDestroy(e->join[i]);
        if (e->aux[i]) (void)hipStreamDestroy(e->aux[i]);
    }
    if (e->fork) (void)hipEventDestroy(e->fork);
    if (e->stream) (void)hipStreamDestroy(e->stream);
}

constexpr size_t kTimedPool = 1024;  // event pairs held before folding

// Zeroes the stage-profile counters, the per-launch earliest start to all ones.
int clearProfile(carl_env* e)
{
    unsigned long long init[kProfWords] = {};
    init[kProfFirst] = ~0ull;
    HIP_TRY(hipMemcpy(e->prof, init, sizeof init, hipMemcpyHostToDevice));
    return CARL_OK;
}

// Adds the durations of the recorded launches to the per-kernel sums (and,
// with the stage profile on, to its launch sums) and frees their events for
// reuse.  Timed launches are on the environment stream.
int foldTiming(carl_env* e)
{
    if (e->timedLaunches == 0) return CARL_OK;
    HIP_TRY(hipStreamSynchronize(e->stream));
    for (size_t i = 0; i < e->timedLaunches; i++) {
        float ms = 0.f;
        HIP_TRY(hipEventElapsedTime(&ms, e->marks[2 * i], e->marks[2 * i + 1]));
        const int k = e->markKernel[i];
        e->kernelMs[k] += ms;
        e->kernelLaunches[k]++;
        if ((e->timing & CARL_TIME_STAGES) && k != CARL_KERNEL_STEP_ENV) e->stageKernelMs[k] += ms;
    }
    e->timedLaunches = 0;
    return CARL_OK;
}

// Timing events of the next timed launch: a start and an end event from a
// pool (created on first use; when all kTimedPool pairs hold unread
// launches, those are folded first), both null when timing is off.
int timedPair(carl_env* e, int kernel, hipEvent_t* begin, hipEvent_t* end)
{
    *begin = *end = nullptr;
    const int want = kernel == CARL_KERNEL_STEP_ENV ? CARL_TIME_PACKING : (CARL_TIME_TICKS | CARL_TIME_STAGES);
    if (!(e->timing & want)) return CARL_OK;
    if (e->timedLaunches == kTimedPool) CARL_TRY(foldTiming(e));
    const size_t slot = 2 * e->timedLaunches;
    while (e->marks.size() < slot + 2) {
        hipEvent_t ev;
        HIP_TRY(hipEventCreate(&ev));
        e->marks.push_back(ev);
    }
    if (e->markKernel.size() <= e->timedLaunches) e->markKernel.resize(e->timedLaunches + 1);
    e->markKernel[e->timedLaunches++] = kernel;
    *begin = e->marks[slot];
    *end = e->marks[slot + 1];
    return CARL_OK;
}

// A tick kernel launch; when timed, its start and end events are recorded
// by the dispatch itself (hipExtLaunchKernelGGL).
template <typename... P, typename... A>
int launchTick(carl_env* e, bool timed, int kernel, void (*k)(P...), dim3 grid, dim3 block, uint32_t lds,
               hipStream_t st, A&&... args)
{
    hipEvent_t b = nullptr, en = nullptr;
    if (timed) {
        const int rc = timedPair(e, kernel, &b, &en);
        if (rc != CARL_OK) return rc;
    }
    hipExtLaunchKernelGGL(k, grid, block, lds, st, b, en, 0, static_cast<P>(args)...);
    return CARL_OK;
}

#define CARL_MARK(expr)                   \
    do {                                  \
        const int rc_ = (expr);           \
        if (rc_ != CARL_OK) return rc_;   \
    } while (0)

// Ticks run as e->tickStreams partitions of the simulations, partition 0 on
// the environment stream and the others on auxiliary streams forked from and
// joined back into it; the partitions share no data within a tick.  With
// windowSims > 0 each partition runs all n ticks in one tick-window launch,
// otherwise four phase kernels per tick.  Timing events bracket partition
// 0's launches.
// Simulations per window workgroup for the next launch: the set size capped
// at a workgroup's cars; until the caller sets it, halved (down to
// kAutoWindowMin) while every partition's workgroups together still fit the
// device's resident window workgroups.
int effectiveWindowSims(const carl_env* e)
{
    if (e->windowSims <= 0) return 0;
    int wsb = std::min(e->windowSims, kWindowBlock / e->nCars);
    if (!e->windowAuto) return wsb;
    const int parts = std::min(e->tickStreams, e->nSim);
    auto blocks = [&](int sims) {
        int total = 0;
        for (int p = 0; p < parts; p++) {
            const int begin = (int)((int64_t)e->nSim * p / parts), end = (int)((int64_t)e->nSim * (p + 1) / parts);
            total += e->grid(end - begin, sims);
        }
        return total;
    };
    while (wsb / 2 >= kAutoWindowMin && blocks(wsb / 2) <= e->windowResident) wsb /= 2;
    return wsb;
}

// Whether a window launch of `ticks` ticks deals its simulations by cost:
// 1v1 or 2v2 on the mesh arena, one partition, workgroups of dealBlockSims
// simulations, all of them full, and at least kDealMinTicks ticks.  (A
// launch of fewer ticks has less tail to even out than the scattered units
// cost it: 2v2 stepped one tick at a time at 131,072 simulations ran 370 ->
// 377 us per launch dealt.)
constexpr int kDealMinTicks = 4;
bool balancedLaunch(const carl_env* e, int ticks)
{
    const int bs = dealBlockSims(e->nCars);
    return e->balance && bs > 0 && !e->native() && e->dealList && std::min(e->tickStreams, e->nSim) == 1
           && effectiveWindowSims(e) == bs && e->nSim % bs == 0 && ticks >= kDealMinTicks;
}

int launchTicks(carl_env* e, int kind, const void* actions, int n)
{
    if (n <= 0) return CARL_OK;
    const int spb = kTickBlock / e->nCars;
    const Dev d = e->dev();
    const int parts = std::min(e->tickStreams, e->nSim);
    SimRange range[kMaxTickStreams];
    hipStream_t stream[kMaxTickStreams];
    for (int p = 0; p < parts; p++) {
        range[p] = SimRange{ (int)((int64_t)e->nSim * p / parts), (int)((int64_t)e->nSim * (p + 1) / parts) };
        stream[p] = p == 0 ? e->stream : e->aux[p - 1];
    }
    if (parts > 1) {
        HIP_TRY(hipEventRecord(e->fork, e->stream));
        for (int p = 1; p < parts; p++) HIP_TRY(hipStreamWaitEvent(stream[p], e->fork, 0));
    }
    if (e->windowSims > 0) {
        const int wsb = effectiveWindowSims(e);
        const bool balanced = balancedLaunch(e, n);
        WindowMap map{};
        if (balanced) {
            // the first balanced launch deals the identity
            const int nU = e->nSim / dealUnitSims(e->nCars);
            const long long l = e->dealLaunches++;
            auto set = [&](long long k, int* base, size_t per) { return base + (size_t)(k % kDealSets) * per; };
            map.inCount = l > 0 ? set(l, e->dealCount, kDealLists) : nullptr;
            map.inList = l > 0 ? set(l, e->dealList, (size_t)kDealClasses * nU) : nullptr;
            map.outCount = set(l + 1, e->dealCount, kDealLists);
            map.outList = set(l + 1, e->dealList, (size_t)kDealClasses * nU);
            map.clearCount = set(l + 2, e->dealCount, kDealLists);
            map.nUnits = nU;
        }
        for (int p = 0; p < parts; p++) {
            const SimRange r = range[p];
            const bool timed = p == 0;
            const int blocks = e->grid(r.end - r.begin, wsb);
            if (timed && (e->timing & CARL_TIME_STAGES)) {
                // the clock sums are divided by one resident-workgroup count
                const int slots = std::min(blocks, e->profResident);
                if (e->profSlots != 0 && e->profSlots != slots) e->profMixed = true;
                e->profSlots = slots;
                CARL_MARK(launchTick(e, timed, CARL_KERNEL_WINDOW, profileKernelFor(e->nCars, balanced),
                                     dim3(blocks),
                                     dim3(kWindowBlock), 0, stream[p], d, e->ws, e->contactScreen, kind, actions,
                                     e->tickCount + 1, n, wsb, r, map, e->prof));
            } else {
                CARL_MARK(launchTick(e, timed, CARL_KERNEL_WINDOW,
                                     e->native() ? tickWindowNativeKernel : windowKernelFor(e->nCars, balanced),
                                     dim3(blocks),
                                     dim3(kWindowBlock), 0, stream[p], d, e->ws, e->contactScreen, kind, actions,
                                     e->tickCount + 1, n, wsb, r, map));
            }
        }
    }
    for (int k = 0; e->windowSims == 0 && k < n; k++) {
        const int tick = e->tickCount + k + 1;
        for (int p = 0; p < parts; p++) {
            const SimRange r = range[p];
            const int sims = r.end - r.begin, cars = sims * e->nCars;
            hipStream_t st = stream[p];
            const bool timed = p == 0;
            CARL_MARK(launchTick(e, timed, CARL_KERNEL_CONTACT, contactKernel, dim3(e->grid(cars, kContactOwners)),
                                 dim3(kContactBlock), 0, st, d, e->ws, e->contactScreen, r));
            CARL_MARK(launchTick(e, timed, CARL_KERNEL_CAR_ARENA, carArenaKernel, dim3(e->grid(cars, kTickBlock)),
                                 dim3(kTickBlock), 0, st, d, e->ws, kind, actions, tick, r));
            CARL_MARK(launchTick(e, timed, CARL_KERNEL_BALL, e->native() ? ballNativeKernel : ballKernel,
                                 dim3(e->grid(sims, kBallOwners)),
                                 dim3(kBallBlock), 0, st, d, tick, r));
            CARL_MARK(launchTick(e, timed, CARL_KERNEL_FINISH, finishKernel, dim3(e->grid(sims, spb)),
                                 dim3(spb * e->nCars), 0, st, d, spb, r));
        }
    }
    HIP_TRY(hipGetLastError());
    for (int p = 1; p < parts; p++) {
        HIP_TRY(hipEventRecord(e->join[p - 1], stream[p]));
        HIP_TRY(hipStreamWaitEvent(e->stream, e->join[p - 1], 0));
    }
    if (e->timing & CARL_TIME_STAGES) {
        const int path = e->windowSims > 0 ? 1 : 2;
        if (e->stagePath != 0 && e->stagePath != path) e->profMixed = true;
        e->stagePath = path;
        e->stageTicks += n;
    }
    e->tickCount += n;
    return CARL_OK;
}

int packObs(carl_env* e, float* out, const bool* mask)
{
    obsKernel<<<e->grid(e->nTotal, packChunkRows(e->obsDim)), kPackBlock, packLdsBytes(e->obsDim), e->stream>>>(
        e->dev(), out, e->obsDim, mask, e->invert, e->normalize, e->prevControls);
    HIP_TRY(hipGetLastError());
    return CARL_OK;
}

int packState(carl_env* e, float* out, int touchWindow, const bool* mask)
{
    stateKernel<<<e->grid(e->nSim, packChunkRows(e->stateDim)), kPackBlock, packLdsBytes(e->stateDim), e->stream>>>(
        e->dev(), out, e->stateDim, touchWindow, e->tickCount, mask);
    HIP_TRY(hipGetLastError());
    return CARL_OK;
}

int packMatch(carl_env* e, const bool* mask)
{
    matchKernel<<<e->grid(e->nSim, 64), 64, 0, e->stream>>>(e->dev(), e->score, e->ticks, e->overtime, mask,
                                                             nullptr, nullptr);
    HIP_TRY(hipGetLastError());
    return CARL_OK;
}

// The outputs a reset changes (observations, state, match state) for the
// simulations of a compacted selection.
int packSelected(carl_env* e, const Selection& sel)
{
    obsListKernel<<<e->grid(e->nTotal, packChunkRows(e->obsDim)), kPackBlock, packLdsBytes(e->obsDim), e->stream>>>(
        e->dev(), e->obs, e->obsDim, e->invert, e->normalize, e->prevControls, sel.list, sel.count);
    HIP_TRY(hipGetLastError());
    stateListKernel<<<e->grid(e->nSim, packChunkRows(e->stateDim)), kPackBlock, packLdsBytes(e->stateDim),
                      e->stream>>>(e->dev(), e->state, e->stateDim, 1, e->tickCount, sel.list, sel.count);
    HIP_TRY(hipGetLastError());
    matchKernel<<<e->grid(e->nSim, 64), 64, 0, e->stream>>>(e->dev(), e->score, e->ticks, e->overtime, nullptr,
                                                             sel.list, sel.count);
    HIP_TRY(hipGetLastError());
    return CARL_OK;
}

int packRewardsDones(carl_env* e)
{
    rewardsDonesKernel<<<e->grid(e->nSim, 64), 64, 0, e->stream>>>(e->dev(), e->tickCount, e->rule(), e->rewards,
                                                                   e->dones, e->tscore, e->tticks, e->tovertime);
    HIP_TRY(hipGetLastError());
    return CARL_OK;
}

int initialPacks(carl_env* e)
{
    CARL_TRY(packObs(e, e->obs, nullptr));
    CARL_TRY(packState(e, e->state, 1, nullptr));
    CARL_TRY(packState(e, e->tstate, 1, nullptr));
    CARL_TRY(packRewardsDones(e));
    CARL_TRY(packMatch(e, nullptr));
    return CARL_OK;
}

int fullReset(carl_env* e)
{
    e->tickCount = 0;
    resetKernel<<<e->grid(e->nSim, 64), 64, 0, e->stream>>>(e->dev(), e->nOrange);
    HIP_TRY(hipGetLastError());
    return initialPacks(e);
}

Selection makeSel(const int64_t* idx, const uint8_t* mask, int n) { return Selection{ idx, mask, n, nullptr, nullptr }; }

int setBallRows(carl_env* e, const float* pos, const float* vel, const float* ang, Selection sel)
{
    if (sel.n == 0) return CARL_OK;
    setBallKernel<<<e->grid(sel.n, 64), 64, 0, e->stream>>>(e->dev(), pos, vel, ang, sel);
    HIP_TRY(hipGetLastError());
    return CARL_OK;
}

int setCarRows(carl_env* e, const float* pos, const float* rot, const float* vel, const float* ang, const void* demoed,
               int byteDemoed, const float* boost, const float* internal, Selection sel)
{
    if (sel.n == 0) return CARL_OK;
    const int n = sel.n * e->nCars;
    setCarKernel<<<e->grid(n, 256), 256, 0, e->stream>>>(e->dev(), pos, rot, vel, ang, demoed, byteDemoed, boost,
                                                          internal, sel);
    HIP_TRY(hipGetLastError());
    refreshKernel<<<e->grid(n, kContactOwners), kContactBlock, 0, e->stream>>>(e->dev(), sel, e->contactScreen);
    HIP_TRY(hipGetLastError());
    return CARL_OK;
}

int setMatchRows(carl_env* e, const int32_t* blue, const int32_t* orange, const int32_t* ticks, Selection sel)
{
    if (sel.n == 0) return CARL_OK;
    setMatchKernel<<<e->grid(sel.n, 64), 64, 0, e->stream>>>(e->dev(), blue, orange, ticks, sel);
    HIP_TRY(hipGetLastError());
    return CARL_OK;
}

int resetPadRows(carl_env* e, Selection sel)
{
    if (sel.n == 0) return CARL_OK;
    resetPadsKernel<<<e->grid(sel.n, 64), 64, 0, e->stream>>>(e->dev(), sel);
    HIP_TRY(hipGetLastError());
    return CARL_OK;
}

int checkEnv(carl_env* e)
{
    if (!e) return fail(CARL_ERR_VALUE, "null environment handle");
    return CARL_OK;
}

int checkSelection(carl_env* e, int n)
{
    if (n < 0 || n > e->nSim) return fail(CARL_ERR_VALUE, "too many simulation_indices");
    return CARL_OK;
}

}  // namespace

// ------------------------------------------------------------------- C-ABI

extern "C" {

const char* carl_last_error(void) { return g_lastError.c_str(); }

int carl_observation_dim(int nCars, int prev) { return observationDim(nCars, prev != 0); }
int carl_state_dim(int nCars) { return stateDim(nCars); }

int carl_env_create(int nSim, int nBlue, int nOrange, int seed, int frameskip, int flags, carl_env** out)
{
    if (!out) return fail(CARL_ERR_VALUE, "null output handle");
    *out = nullptr;
    if (frameskip < 1) return fail(CARL_ERR_VALUE, "frameskip must be at least 1");
    if (nSim < 1) return fail(CARL_ERR_VALUE, "n_sim must be at least 1");
    if (nBlue < 0 || nOrange < 0 || nBlue + nOrange < 1) return fail(CARL_ERR_VALUE, "need at least one car");
    if (nBlue > 4 || nOrange > 4) return fail(CARL_ERR_VALUE, "at most 4 cars per team (kickoff spawns)");
    CARL_TRY(checkSizes(nSim, nBlue + nOrange));

    // the host build and its errors come before any device work
    DeviceArena* arena = nullptr;
    CARL_TRY(acquireArena(&arena));

    carl_env* e = new carl_env();
    e->arena = arena;
    e->nSim = nSim; e->nBlue = nBlue; e->nOrange = nOrange; e->nCars = nBlue + nOrange;
    e->nTotal = nSim * e->nCars; e->seed = seed; e->frameskip = frameskip;
    e->invert = (flags & CARL_FLAG_INVERT_ORANGE) != 0;
    e->normalize = (flags & CARL_FLAG_NORMALIZE) != 0;
    e->prevControls = (flags & CARL_FLAG_PREVIOUS_CONTROLS) != 0;
    e->obsDim = observationDim(e->nCars, e->prevControls);
    e->stateDim = stateDim(e->nCars);

    auto bail = [&](int rc) {
        freeAll(e);
        delete e;
        return rc;
    };
    if (hipStreamCreateWithFlags(&e->stream, hipStreamNonBlocking) != hipSuccess)
        return bail(fail(CARL_ERR_RUNTIME, "hipStreamCreate failed"));
    if (hipEventCreateWithFlags(&e->fork, hipEventDisableTiming) != hipSuccess)
        return bail(fail(CARL_ERR_RUNTIME, "hipEventCreate failed"));
    for (int i = 0; i < kMaxTickStreams - 1; i++) {
        if (hipStreamCreateWithFlags(&e->aux[i], hipStreamNonBlocking) != hipSuccess
            || hipEventCreateWithFlags(&e->join[i], hipEventDisableTiming) != hipSuccess)
            return bail(fail(CARL_ERR_RUNTIME, "hipStreamCreate failed"));
    }
    {
        int device = 0, cus = 0, perCu = 0;
        if (hipGetDevice(&device) != hipSuccess
            || hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, device) != hipSuccess
            || hipOccupancyMaxActiveBlocksPerMultiprocessor(
                   &perCu, windowKernelFor(e->nCars, false), kWindowBlock, 0) != hipSuccess)
            return bail(fail(CARL_ERR_RUNTIME, "window kernel occupancy query failed"));
        e->windowResident = perCu * cus;
    }
    const size_t nT = (size_t)e->nTotal, nS = (size_t)nSim;
    int rc = CARL_OK;
    rc = rc ? rc : devAlloc(&e->car, (size_t)CARL_CAR_FIELDS * tiledItems(e->nTotal));
    rc = rc ? rc : devAlloc(&e->sim, (size_t)CARL_SIM_FIELDS * tiledItems(nSim));
    rc = rc ? rc : devAlloc(&e->obs, nT * e->obsDim);
    rc = rc ? rc : devAlloc(&e->tobs, nT * e->obsDim);
    rc = rc ? rc : devAlloc(&e->state, nS * e->stateDim);
    rc = rc ? rc : devAlloc(&e->tstate, nS * e->stateDim);
    rc = rc ? rc : devAlloc(&e->rewards, nS);
    rc = rc ? rc : devAlloc(&e->dones, nS);
    rc = rc ? rc : devAlloc(&e->overtime, nS);
    rc = rc ? rc : devAlloc(&e->tovertime, nS);
    rc = rc ? rc : devAlloc(&e->score, nS);
    rc = rc ? rc : devAlloc(&e->ticks, nS);
    rc = rc ? rc : devAlloc(&e->tscore, nS);
    rc = rc ? rc : devAlloc(&e->tticks, nS);
    rc = rc ? rc : devAlloc(&e->actions, nT * 7);
    rc = rc ? rc : devAlloc(&e->cactions, nT * 7);
    rc = rc ? rc : devAlloc(&e->ws, (size_t)kWsPlanes * tiledItems(e->nTotal));
    rc = rc ? rc : devAlloc(&e->rowList, nS + 1);
    if (dealBlockSims(e->nCars) > 0 && nS % dealBlockSims(e->nCars) == 0) {
        rc = rc ? rc : devAlloc(&e->dealCount, (size_t)kDealSets * kDealLists);
        rc = rc ? rc : devAlloc(&e->dealList, (size_t)kDealSets * kDealClasses * (nS / dealUnitSims(e->nCars)));
    }
    if (e->native()) rc = rc ? rc : devAlloc(&e->ballScratch, (size_t)kNativeMaxContacts * kNativeSlotWords * nS);
    if (rc) return bail(rc);

    rc = fullReset(e);
    if (rc) return bail(rc);
    *out = e;
    return CARL_OK;
}

int carl_env_destroy(carl_env* e)
{
    if (!e) return CARL_OK;
    if (e->stream) (void)hipStreamSynchronize(e->stream);
    freeAll(e);
    delete e;
    return CARL_OK;
}

void* carl_env_stream(carl_env* e) { return e ? (void*)e->stream : nullptr; }

int carl_env_synchronize(carl_env* e)
{
    CARL_TRY(checkEnv(e));
    HIP_TRY(hipStreamSynchronize(e->stream));
    return CARL_OK;
}

int carl_env_tick(carl_env* e, int kind, const void* actions, int n)
{
    CARL_TRY(checkEnv(e));
    if (kind < CARL_ACTIONS_DISCRETE || kind > CARL_ACTIONS_DIRECT) return fail(CARL_ERR_VALUE, "unknown action kind");
    if (!actions) return fail(CARL_ERR_VALUE, "null actions");
    return launchTicks(e, kind, actions, n);
}

int carl_env_reset_dones(carl_env* e)
{
    CARL_TRY(checkEnv(e));
    resetDonesKernel<<<e->grid(e->nSim, 64), 64, 0, e->stream>>>(e->dev(), e->nOrange, e->tickCount, e->rule());
    HIP_TRY(hipGetLastError());
    return CARL_OK;
}

int carl_env_step(carl_env* e, int kind, const void* actions)
{
    CARL_TRY(checkEnv(e));
    if (!actions) return fail(CARL_ERR_VALUE, "null actions");
    uint32_t* keep = nullptr;
    if (kind == CARL_ACTIONS_DISCRETE) keep = (uint32_t*)e->actions;
    else if (kind == CARL_ACTIONS_CONTINUOUS) keep = (uint32_t*)e->cactions;
    else if (kind != CARL_ACTIONS_DIRECT) return fail(CARL_ERR_VALUE, "unknown action kind");
    CARL_TRY(launchTicks(e, kind, actions, e->frameskip));
    StepIO io{};
    io.rewards = e->rewards; io.tstate = e->tstate; io.tobs = e->tobs; io.obs = e->obs; io.state = e->state;
    io.dones = e->dones; io.tovertime = e->tovertime; io.overtime = e->overtime;
    io.tscore = e->tscore; io.tticks = e->tticks; io.score = e->score; io.ticks = e->ticks;
    io.actions = (const uint32_t*)actions;
    io.actionCopy = keep == actions ? nullptr : keep;
    io.obsDim = e->obsDim; io.stateDim = e->stateDim;
    io.invert = e->invert; io.normalize = e->normalize; io.prev = e->prevControls;
    io.frameskip = e->frameskip; io.tickCount = e->tickCount; io.nOrange = e->nOrange;
    io.rule = e->rule();
    const size_t lds = stepLdsBytes(e->obsDim, e->stateDim);
    CARL_TRY(launchTick(e, true, CARL_KERNEL_STEP_ENV, stepEnvKernel, dim3(e->grid(e->nSim, kStepSims)),
                        dim3(kPackBlock), (uint32_t)lds, e->stream, e->dev(), io));
    HIP_TRY(hipGetLastError());
    return CARL_OK;
}

int carl_env_reset(carl_env* e)
{
    CARL_TRY(checkEnv(e));
    return fullReset(e);
}

int carl_env_set_ball(carl_env* e, const float* pos, const float* vel, const float* ang, const int64_t* idx, int n)
{
    CARL_TRY(checkEnv(e));
    if (!idx) n = e->nSim;
    CARL_TRY(checkSelection(e, n));
    if (n > 0 && (!pos || !vel || !ang)) return fail(CARL_ERR_VALUE, "null ball input");
    CARL_TRY(setBallRows(e, pos, vel, ang, makeSel(idx, nullptr, n)));
    CARL_TRY(packObs(e, e->obs, nullptr));
    CARL_TRY(packState(e, e->state, 1, nullptr));
    CARL_TRY(packState(e, e->tstate, 1, nullptr));
    return CARL_OK;
}

int carl_env_set_car(carl_env* e, const float* pos, const float* rot, const float* vel, const float* ang,
                     const void* demoed, int byteDemoed, const float* boost, const float* internal, const int64_t* idx,
                     int n)
{
    CARL_TRY(checkEnv(e));
    if (!idx) n = e->nSim;
    CARL_TRY(checkSelection(e, n));
    if (n > 0 && (!pos || !rot || !vel || !ang || !demoed)) return fail(CARL_ERR_VALUE, "null car input");
    CARL_TRY(setCarRows(e, pos, rot, vel, ang, demoed, byteDemoed, boost, internal, makeSel(idx, nullptr, n)));
    CARL_TRY(packObs(e, e->obs, nullptr));
    CARL_TRY(packState(e, e->state, 1, nullptr));
    CARL_TRY(packState(e, e->tstate, 1, nullptr));
    return CARL_OK;
}

int carl_env_apply_reset(carl_env* e, const float* bpos, const float* bvel, const float* bang, const float* cpos,
                         const float* crot, const float* cvel, const float* cang, const void* demoed, int byteDemoed,
                         const float* boost, const float* internal, const int32_t* blue, const int32_t* orange,
                         const int32_t* ticks, const int64_t* idx, int n, const uint8_t* mask)
{
    CARL_TRY(checkEnv(e));
    if (idx && mask) return fail(CARL_ERR_VALUE, "specify reset_mask or simulation_indices, not both");
    if (!idx) n = e->nSim;
    CARL_TRY(checkSelection(e, n));
    const bool hasMatch = blue != nullptr;
    if (hasMatch != (orange != nullptr) || hasMatch != (ticks != nullptr))
        return fail(CARL_ERR_VALUE, "blue_score, orange_score and episode_ticks must be supplied together");
    if (n == 0) return CARL_OK;
    if (!bpos || !bvel || !bang || !cpos || !crot || !cvel || !cang || !demoed)
        return fail(CARL_ERR_VALUE, "null reset input");
    Selection sel = makeSel(idx, mask, n);
    if (mask) {
        // the selected rows, compacted on the device: every kernel below
        // runs over them only
        sel.list = e->rowList;
        sel.count = e->rowList + e->nSim;
        clearCountKernel<<<1, 1, 0, e->stream>>>(e->rowList + e->nSim);
        compactMaskKernel<<<e->grid(n, kCompactBlock * kCompactRows), kCompactBlock, 0, e->stream>>>(
            mask, n, e->rowList, e->rowList + e->nSim);
        HIP_TRY(hipGetLastError());
    }
    CARL_TRY(resetPadRows(e, sel));
    CARL_TRY(setBallRows(e, bpos, bvel, bang, sel));
    CARL_TRY(setCarRows(e, cpos, crot, cvel, cang, demoed, byteDemoed, boost, internal, sel));
    if (hasMatch) CARL_TRY(setMatchRows(e, blue, orange, ticks, sel));
    if (mask) return packSelected(e, sel);
    CARL_TRY(packObs(e, e->obs, nullptr));
    CARL_TRY(packState(e, e->state, 1, nullptr));
    CARL_TRY(packMatch(e, nullptr));
    return CARL_OK;
}

int carl_env_set_match(carl_env* e, const int32_t* blue, const int32_t* orange, const int32_t* ticks,
                       const int64_t* idx, int n)
{
    CARL_TRY(checkEnv(e));
    if (!idx) n = e->nSim;
    CARL_TRY(checkSelection(e, n));
    if (n > 0 && (!blue || !orange || !ticks)) return fail(CARL_ERR_VALUE, "null match input");
    return setMatchRows(e, blue, orange, ticks, makeSel(idx, nullptr, n));
}

int carl_env_reset_pads(carl_env* e, const int64_t* idx, int n)
{
    CARL_TRY(checkEnv(e));
    if (!idx) n = e->nSim;
    CARL_TRY(checkSelection(e, n));
    return resetPadRows(e, makeSel(idx, nullptr, n));
}

int carl_env_buffer(carl_env* e, int id, void** data, int64_t* shape, int* ndim, int* dtype)
{
    CARL_TRY(checkEnv(e));
    if (!data || !shape || !ndim || !dtype) return fail(CARL_ERR_VALUE, "null output pointer");
    const int64_t nS = e->nSim, nC = e->nCars;
    auto set = [&](void* p, int nd, int64_t a, int64_t b, int64_t c, int dt) {
        *data = p; *ndim = nd; shape[0] = a; shape[1] = b; shape[2] = c; *dtype = dt;
        return CARL_OK;
    };
    switch (id) {
    case CARL_BUF_OBS: return set(e->obs, 3, nS, nC, e->obsDim, CARL_DTYPE_F32);
    case CARL_BUF_TRANSITION_OBS: return set(e->tobs, 3, nS, nC, e->obsDim, CARL_DTYPE_F32);
    case CARL_BUF_STATE: return set(e->state, 2, nS, e->stateDim, 0, CARL_DTYPE_F32);
    case CARL_BUF_TRANSITION_STATE: return set(e->tstate, 2, nS, e->stateDim, 0, CARL_DTYPE_F32);
    case CARL_BUF_ACTIONS: return set(e->actions, 3, nS, nC, 7, CARL_DTYPE_I32);
    case CARL_BUF_CONTINUOUS_ACTIONS: return set(e->cactions, 3, nS, nC, 7, CARL_DTYPE_F32);
    case CARL_BUF_REWARDS: return set(e->rewards, 1, nS, 0, 0, CARL_DTYPE_F32);
    case CARL_BUF_DONES: return set(e->dones, 1, nS, 0, 0, CARL_DTYPE_BOOL);
    case CARL_BUF_SCORE_DIFFERENCE: return set(e->score, 1, nS, 0, 0, CARL_DTYPE_I32);
    case CARL_BUF_EPISODE_TICKS: return set(e->ticks, 1, nS, 0, 0, CARL_DTYPE_I32);
    case CARL_BUF_TRANSITION_SCORE_DIFFERENCE: return set(e->tscore, 1, nS, 0, 0, CARL_DTYPE_I32);
    case CARL_BUF_TRANSITION_EPISODE_TICKS: return set(e->tticks, 1, nS, 0, 0, CARL_DTYPE_I32);
    case CARL_BUF_OVERTIME: return set(e->overtime, 1, nS, 0, 0, CARL_DTYPE_BOOL);
    case CARL_BUF_TRANSITION_OVERTIME: return set(e->tovertime, 1, nS, 0, 0, CARL_DTYPE_BOOL);
    default: return fail(CARL_ERR_VALUE, "unknown buffer id");
    }
}

int carl_env_set_param(carl_env* e, int p, int v)
{
    CARL_TRY(checkEnv(e));
    switch (p) {
    case CARL_PARAM_MAX_TICKS:
        if (v < 1) return fail(CARL_ERR_VALUE, "max_ticks must be at least 1");
        e->maxTicks = v;
        return CARL_OK;
    case CARL_PARAM_OVERTIME_TIMEOUT_TICKS:
        if (v < 1) return fail(CARL_ERR_VALUE, "overtime_timeout_ticks must be at least 1");
        e->overtimeTicks = v;
        return CARL_OK;
    case CARL_PARAM_NO_TOUCH_TIMEOUT_TICKS:
        if (v < 0) return fail(CARL_ERR_VALUE, "no_touch_timeout_ticks must be non-negative");
        e->noTouchTicks = v;
        return CARL_OK;
    case CARL_PARAM_FRAMESKIP:
        if (v < 1) return fail(CARL_ERR_VALUE, "frameskip must be at least 1");
        e->frameskip = v;
        return CARL_OK;
    case CARL_PARAM_TICK_STREAMS:
        if (v < 1 || v > kMaxTickStreams) return fail(CARL_ERR_VALUE, "tick_streams must be in [1, 4]");
        e->tickStreams = v;
        return CARL_OK;
    case CARL_PARAM_CONTACT_SCREEN:
        if (v != 0 && v != 1) return fail(CARL_ERR_VALUE, "contact_screen must be 0 or 1");
        e->contactScreen = v;
        return CARL_OK;
    case CARL_PARAM_TICK_WINDOW:
        if (v < 0 || v > kWindowBlock) return fail(CARL_ERR_VALUE, "tick_window must be in [0, 128]");
        e->windowSims = v;
        e->windowAuto = false;
        return CARL_OK;
    case CARL_PARAM_TICK_BALANCE:
        if (v != 0 && v != 1) return fail(CARL_ERR_VALUE, "tick_balance must be 0 or 1");
        e->balance = v;
        return CARL_OK;
    default: return fail(CARL_ERR_VALUE, "parameter is read-only or unknown");
    }
}

int carl_env_get_param(carl_env* e, int p, int* v)
{
    CARL_TRY(checkEnv(e));
    if (!v) return fail(CARL_ERR_VALUE, "null output pointer");
    switch (p) {
    case CARL_PARAM_MAX_TICKS: *v = e->maxTicks; break;
    case CARL_PARAM_OVERTIME_TIMEOUT_TICKS: *v = e->overtimeTicks; break;
    case CARL_PARAM_NO_TOUCH_TIMEOUT_TICKS: *v = e->noTouchTicks; break;
    case CARL_PARAM_FRAMESKIP: *v = e->frameskip; break;
    case CARL_PARAM_N_SIM: *v = e->nSim; break;
    case CARL_PARAM_N_CARS: *v = e->nCars; break;
    case CARL_PARAM_OBS_DIM: *v = e->obsDim; break;
    case CARL_PARAM_ACT_DIM: *v = e->nCars * 7; break;
    case CARL_PARAM_STATE_DIM: *v = e->stateDim; break;
    case CARL_PARAM_TICK_COUNT: *v = e->tickCount; break;
    case CARL_PARAM_N_BLUE: *v = e->nBlue; break;
    case CARL_PARAM_TICK_STREAMS: *v = e->tickStreams; break;
    case CARL_PARAM_CONTACT_SCREEN: *v = e->contactScreen; break;
    case CARL_PARAM_TICK_WINDOW: *v = e->windowSims; break;
    case CARL_PARAM_TICK_WINDOW_LAUNCH: *v = effectiveWindowSims(e); break;
    case CARL_PARAM_NATIVE_ARENA: *v = e->native(); break;
    case CARL_PARAM_TICK_BALANCE: *v = e->balance; break;
    case CARL_PARAM_TICK_BALANCED_LAUNCH: *v = balancedLaunch(e, e->frameskip); break;
    default: return fail(CARL_ERR_VALUE, "unknown parameter");
    }
    return CARL_OK;
}

int carl_env_enable_timing(carl_env* e, int enable)
{
    CARL_TRY(checkEnv(e));
    HIP_TRY(hipStreamSynchronize(e->stream));
    if ((enable & CARL_TIME_STAGES) && e->native())
        return fail(CARL_ERR_VALUE, "the stage profile does not cover the native arena meshes");
    e->timing = enable & (CARL_TIME_TICKS | CARL_TIME_PACKING | CARL_TIME_STAGES);
    e->timedLaunches = 0;
    for (int k = 0; k < CARL_TICK_KERNELS; k++) {
        e->kernelMs[k] = e->stageKernelMs[k] = 0.0;
        e->kernelLaunches[k] = 0;
    }
    e->stageTicks = e->stagePath = e->profSlots = 0;
    e->profMixed = false;
    if (e->timing & CARL_TIME_STAGES) {
        if (!e->prof) CARL_TRY(devAlloc(&e->prof, kProfWords));
        CARL_TRY(clearProfile(e));
        int device = 0, cus = 0, perCu = 0, khz = 0;
        HIP_TRY(hipGetDevice(&device));
        HIP_TRY(hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, device));
        HIP_TRY(hipDeviceGetAttribute(&khz, hipDeviceAttributeWallClockRate, device));
        HIP_TRY(hipOccupancyMaxActiveBlocksPerMultiprocessor(&perCu, profileKernelFor(e->nCars, false), kWindowBlock,
                                                             0));
        if (khz <= 0 || perCu <= 0) return fail(CARL_ERR_RUNTIME, "no wall-clock rate or window occupancy");
        e->profResident = perCu * cus;
        e->clockMHz = khz / 1000.0;
    }
    return CARL_OK;
}

int carl_env_tick_timing(carl_env* e, double* kernelMs, int* launches)
{
    CARL_TRY(checkEnv(e));
    if (!kernelMs || !launches) return fail(CARL_ERR_VALUE, "null output pointer");
    CARL_TRY(foldTiming(e));
    HIP_TRY(hipStreamSynchronize(e->stream));
    for (int k = 0; k < CARL_TICK_KERNELS; k++) {
        kernelMs[k] = e->kernelMs[k];
        launches[k] = e->kernelLaunches[k];
        e->kernelMs[k] = 0.0;
        e->kernelLaunches[k] = 0;
    }
    return CARL_OK;
}

int carl_env_stage_timing(carl_env* e, double* stageUs, double* lastUs, double* spanUs, double* launchUs, int* ticks)
{
    CARL_TRY(checkEnv(e));
    if (!stageUs || !lastUs || !spanUs || !launchUs || !ticks) return fail(CARL_ERR_VALUE, "null output pointer");
    if (!(e->timing & CARL_TIME_STAGES)) return fail(CARL_ERR_VALUE, "the stage profile is not enabled");
    CARL_TRY(foldTiming(e));
    HIP_TRY(hipStreamSynchronize(e->stream));
    const bool mixed = e->profMixed;
    const int n = e->stageTicks, path = e->stagePath, slots = e->profSlots;
    unsigned long long clocks[kProfWords] = {};
    HIP_TRY(hipMemcpy(clocks, e->prof, sizeof clocks, hipMemcpyDeviceToHost));
    double kernelMs[CARL_TICK_KERNELS];
    std::copy(e->stageKernelMs, e->stageKernelMs + CARL_TICK_KERNELS, kernelMs);
    // start the next period
    CARL_TRY(clearProfile(e));
    std::fill(e->stageKernelMs, e->stageKernelMs + CARL_TICK_KERNELS, 0.0);
    e->stageTicks = e->stagePath = e->profSlots = 0;
    e->profMixed = false;
    if (mixed) return fail(CARL_ERR_VALUE, "the tick launch shape changed during the stage profile");
    *ticks = n;
    *launchUs = *spanUs = 0.0;
    std::fill(stageUs, stageUs + CARL_STAGES, 0.0);
    std::fill(lastUs, lastUs + CARL_STAGES + 1, 0.0);
    if (n == 0) return CARL_OK;
    if (path == 1) {
        const double us = 1.0 / (e->clockMHz * n);  // clock ticks -> us per tick
        // workgroup time of each phase over the workgroups resident at once
        for (int s = 0; s < CARL_STAGES; s++) {
            stageUs[s] = clocks[kProfStages + s] * us / slots;
            lastUs[s] = clocks[kProfLast + s] * us;
        }
        lastUs[CARL_STAGES] = clocks[kProfLastDelay] * us;
        *spanUs = clocks[kProfSpan] * us;
        *launchUs = kernelMs[CARL_KERNEL_WINDOW] * 1e3 / n;
    } else {
        // one phase kernel per stage; the boost pads run in the finish kernel
        const int kernel[CARL_STAGES - 1] = { CARL_KERNEL_CONTACT, CARL_KERNEL_CAR_ARENA, CARL_KERNEL_BALL,
                                              CARL_KERNEL_FINISH };
        for (int s = 0; s < CARL_STAGES - 1; s++) {
            stageUs[s] = lastUs[s] = kernelMs[kernel[s]] * 1e3 / n;
            *launchUs += stageUs[s];
        }
        *spanUs = *launchUs;
    }
    return CARL_OK;
}

const char* carl_stage_name(int stage)
{
    static const char* names[CARL_STAGES] = { "contact", "car-arena", "ball", "finish", "boost-pads" };
    return stage >= 0 && stage < CARL_STAGES ? names[stage] : "";
}

const char* carl_tick_kernel_name(int kernel)
{
    static const char* names[CARL_TICK_KERNELS] = { "contactKernel", "carArenaKernel", "ballKernel", "finishKernel",
                                                     "tickWindowKernel", "stepEnvKernel" };
    return kernel >= 0 && kernel < CARL_TICK_KERNELS ? names[kernel] : "";
}

int carl_env_export_state(carl_env* e, uint32_t* car, uint32_t* sim, int* tick)
{
    CARL_TRY(checkEnv(e));
    HIP_TRY(hipStreamSynchronize(e->stream));
    // device tiles of 64 items -> planes (field f, item i at f * n + i)
    auto untile = [](const uint32_t* dev, uint32_t* out, int fields, int n) -> int {
        std::vector<uint32_t> tiles((size_t)fields * tiledItems(n));
        HIP_TRY(hipMemcpy(tiles.data(), dev, tiles.size() * sizeof(uint32_t), hipMemcpyDeviceToHost));
        for (int f = 0; f < fields; f++)
            for (int i = 0; i < n; i++) out[(size_t)f * n + i] = tiles[tiledWord(f, i, fields)];
        return CARL_OK;
    };
    if (car) CARL_TRY(untile(e->car, car, CARL_CAR_FIELDS, e->nTotal));
    if (sim) CARL_TRY(untile(e->sim, sim, CARL_SIM_FIELDS, e->nSim));
    if (tick) *tick = e->tickCount;
    return CARL_OK;
}

int carl_env_import_state(carl_env* e, const uint32_t* car, const uint32_t* sim, int tick)
{
    CARL_TRY(checkEnv(e));
    if (!car || !sim) return fail(CARL_ERR_VALUE, "null state buffer");
    HIP_TRY(hipStreamSynchronize(e->stream));
    // planes -> device tiles of 64 items (the padding items stay zero)
    auto tile = [](const uint32_t* in, uint32_t* dev, int fields, int n) -> int {
        std::vector<uint32_t> tiles((size_t)fields * tiledItems(n), 0u);
        for (int f = 0; f < fields; f++)
            for (int i = 0; i < n; i++) tiles[tiledWord(f, i, fields)] = in[(size_t)f * n + i];
        HIP_TRY(hipMemcpy(dev, tiles.data(), tiles.size() * sizeof(uint32_t), hipMemcpyHostToDevice));
        return CARL_OK;
    };
    CARL_TRY(tile(car, e->car, CARL_CAR_FIELDS, e->nTotal));
    CARL_TRY(tile(sim, e->sim, CARL_SIM_FIELDS, e->nSim));
    e->tickCount = tick;
    return CARL_OK;
}

int carl_env_pack_rewards_dones(carl_env* e)
{
    CARL_TRY(checkEnv(e));
    return packRewardsDones(e);
}

int carl_env_pack_transition_state(carl_env* e, int touchWindow)
{
    CARL_TRY(checkEnv(e));
    if (touchWindow < 1) return fail(CARL_ERR_VALUE, "touch window must be at least 1");
    return packState(e, e->tstate, touchWindow, nullptr);
}

int carl_env_pack_transition_obs(carl_env* e)
{
    CARL_TRY(checkEnv(e));
    return packObs(e, e->tobs, e->dones);
}

int carl_env_pack_match_state(carl_env* e, const uint8_t* mask)
{
    CARL_TRY(checkEnv(e));
    return packMatch(e, (const bool*)mask);
}

int carl_env_pack_obs(carl_env* e, const uint8_t* mask)
{
    CARL_TRY(checkEnv(e));
    return packObs(e, e->obs, (const bool*)mask);
}

int carl_env_pack_state(carl_env* e, const uint8_t* mask)
{
    CARL_TRY(checkEnv(e));
    return packState(e, e->state, 1, (const bool*)mask);
}

int carl_env_set_actions(carl_env* e, int kind, const void* actions)
{
    CARL_TRY(checkEnv(e));
    if (!actions) return fail(CARL_ERR_VALUE, "null actions");
    void* dst = nullptr;
    if (kind == CARL_ACTIONS_DISCRETE) dst = e->actions;
    else if (kind == CARL_ACTIONS_CONTINUOUS) dst = e->cactions;
    else return fail(CARL_ERR_VALUE, "actions kind must be discrete or continuous");
    HIP_TRY(hipMemcpyAsync(dst, actions, sizeof(uint32_t) * 7 * (size_t)e->nTotal, hipMemcpyDeviceToDevice,
                           e->stream));
    return CARL_OK;
}

int carl_exclusive_scan_i32(const int32_t* in, int32_t* out, int n, void* stream)
{
    if (n < 0) return fail(CARL_ERR_VALUE, "negative length");
    if (n > 0 && (!in || !out)) return fail(CARL_ERR_VALUE, "null scan buffer");
    return runScan(in, out, n, (hipStream_t)stream);
}

int carl_exclusive_scan_i32_noalloc(const int32_t* in, int32_t* out, int n, void* stream)
{
    if (n < 0) return fail(CARL_ERR_VALUE, "negative length");
    if (n > kScanNoAllocMaxItems)
        return fail(CARL_ERR_VALUE, "scan length exceeds the no-allocation maximum of "
                                        + std::to_string(kScanNoAllocMaxItems) + " items");
    if (n > 0 && (!in || !out)) return fail(CARL_ERR_VALUE, "null scan buffer");
    if (n == 0) return CARL_OK;
    int32_t* work = nullptr;
    CARL_TRY(scratchOnCurrentDevice(&work));
    if (scanWorkWords(n) > kScanScratchWords) return fail(CARL_ERR_VALUE, "scan scratch too small");
    return runScanInto(in, out, n, (hipStream_t)stream, work);
}

}  // extern "C"
