// constants.h - physical constants, capacities and tables of the CARL step.
//
// Values and their float evaluation order restate the reference constants
// (include/RLConstants.cuh:5-278, include/Physics/BoostPads.cuh:14-56,
// include/Physics/BallArena/Contact.cuh:28-37) - they define the game, so
// they must be identical.  The kickoff permutation table is generated from
// its closed form instead of being tabulated.
#pragma once

#include "dmath.h"

namespace carl {

constexpr float kPi2 = kPi / 2;
constexpr float kPi4 = kPi / 4;
constexpr float kSqrtHalf = 0.7071067811865475244f;
constexpr float kFltEps = 1.192092896e-07f;
constexpr float kFltMax = 3.402823466e+38f;

// arena and broadphase grid
constexpr V3 kArenaMin{ -4108.f, -6000.f, -14.f };
constexpr V3 kArenaMax{ 4108.f, 6000.f, 2076.f };
constexpr int kGridX = 48, kGridY = 48, kGridZ = 10;
constexpr int kCells = kGridX * kGridY * kGridZ;
constexpr float kCellX = (kArenaMax.x - kArenaMin.x) / 48.f;
constexpr float kCellY = (kArenaMax.y - kArenaMin.y) / 48.f;
constexpr float kCellZ = (kArenaMax.z - kArenaMin.z) / 10.f;
constexpr float kBoundaryEdge = 2.f * kPi;
// ball candidate grid: cubic cells over the broadphase box; a cell lists every
// triangle whose box comes within ball reach (+1 uu) of the cell.  64 uu cells
// list about half the triangles of 128 uu ones near the curved walls (1.46 M
// references, 210 MB, against 0.26 M); the cars' contact search, which walks
// the same lists, runs 3.5% faster per step once cars have spread to the walls.
constexpr float kFineCell = 64.f;
constexpr int kFineX = 129, kFineY = 188, kFineZ = 33;   // ceil(extent / kFineCell)
constexpr int kFineCells = kFineX * kFineY * kFineZ;
static_assert(kFineX * kFineCell >= kArenaMax.x - kArenaMin.x && kFineY * kFineCell >= kArenaMax.y - kArenaMin.y &&
                  kFineZ * kFineCell >= kArenaMax.z - kArenaMin.z,
              "ball grid must cover the broadphase box");
// car candidate grid: the same lists for the cars' contact search, in 32 uu
// cells and with the car's own reach (every car test stays within 76.6 uu of
// the car's centre, engine.hip), so a car near a curved wall walks about 30%
// fewer candidates than in the ball's lists.  Each list is triangle indices
// only (6.67 M references, 27 MB).
constexpr float kCarCell = 32.f;
constexpr float kCarGridReach = 78.f;
constexpr int kCarX = 257, kCarY = 375, kCarZ = 66;   // ceil(extent / kCarCell)
constexpr int kCarCells = kCarX * kCarY * kCarZ;
static_assert(kCarX * kCarCell >= kArenaMax.x - kArenaMin.x && kCarY * kCarCell >= kArenaMax.y - kArenaMin.y &&
                  kCarZ * kCarCell >= kArenaMax.z - kArenaMin.z,
              "car grid must cover the broadphase box");

// car
constexpr V3 kHalf{ 60.186455f, 43.282655f, 19.262505f };
constexpr float kCarMargin = 1.932955f;
constexpr V3 kHitboxOffset{ 13.87566f, 0.f, 20.755f };
constexpr float kCarRestZ = 17.f;
constexpr float kCarRespawnZ = 36.f;
constexpr float kBallRestZ = 93.15f;
constexpr float kBallRadius = 91.25f;

constexpr int kPads = 34;
constexpr float kBoostMax = 100.f;
constexpr float kBoostSpawn = kBoostMax / 3.f;

constexpr int kWheels = 4;
constexpr float kFrontRadius = 12.5f, kBackRadius = 15.f;
constexpr float kFrontRest = 26.755f, kBackRest = 25.055f;
constexpr float kMaxTravel = 12.f;
constexpr float kSuspSub = 2.5f;
constexpr float kFrontX = 37.3743f, kFrontY = 25.9f, kBackX = -47.6257f, kBackY = 29.5f;
constexpr float kFrontRay = kFrontRest + kMaxTravel + kFrontRadius - kSuspSub;
constexpr float kBackRay = kBackRest + kMaxTravel + kBackRadius - kSuspSub;
enum : int { kSrcNone = 0, kSrcArena = 1, kSrcCar = 2, kSrcBall = 3 };

constexpr int kMaxTriHits = 32;
constexpr int kMaxManifold = 4;
constexpr float kAngMotionThresh = kPi4;
constexpr float kWorldRestitution = 0.3f;
constexpr float kWorldFriction = 0.3f;
constexpr float kContactBreak = 2.03122735f;

constexpr int kTicksPerSecond = 120;
constexpr float kDt = 1.f / kTicksPerSecond;
constexpr int kRegulationTicks = 5 * 60 * kTicksPerSecond;
constexpr float kCarMass = 180.f;
constexpr float kCarInvMass = 1.f / kCarMass;
constexpr float kCarMaxSpeed = 2300.f;
constexpr float kCarMaxAng = 5.5f;
constexpr V3 kCarInvInertia{ 1.f / 134665.94f, 1.f / 239607.22f, 1.f / 329747.90f };
constexpr V3 kGravity{ 0.f, 0.f, -650.f };

constexpr int kSolverIters = 10;
constexpr float kContactErp = 0.8f;
constexpr float kWarmStart = 0.85f;
constexpr float kLinearSlop = 0.f;
constexpr float kSplitTurnErp = 0.1f;
constexpr float kSplitPenThresh = 1.0e30f;
constexpr float kRestitutionThresh = 10.f;

constexpr float kSuspStiffness = 500.f;
constexpr float kDampCompression = 25.f, kDampRelaxation = 40.f;
constexpr float kSuspScaleFront = 35.75f, kSuspScaleBack = 54.265f;
constexpr float kPushbackErp = 0.2f;
constexpr float kPushbackDtFirst = 1.f / 60.f;
constexpr float kStoppingVel = 25.f;
constexpr float kAutorollForce = 100.f, kAutorollTorque = 80.f;

constexpr float kJumpAccel = 4375.f / 3.f;
constexpr float kJumpImmediate = 875.f / 3.f;
constexpr float kJumpMinTime = 0.025f;
constexpr float kJumpResetPad = 1.f / 40.f;
constexpr float kJumpMaxTime = 0.2f;
constexpr float kDoubleJumpWindow = 1.25f;
constexpr float kFlipZDamp = 0.35f, kFlipZDampStart = 0.15f, kFlipZDampEnd = 0.21f;
constexpr float kFlipTorqueTime = 0.65f, kFlipPitchlockExtra = 0.3f;
constexpr float kFlipInitialVel = 500.f;
constexpr float kFlipTorqueX = 260.f, kFlipTorqueY = 224.f;
constexpr float kFlipFwdScale = 1.f, kFlipSideScale = 1.9f, kFlipBackScale = 2.5f;
constexpr float kFlipBackX = 16.f / 15.f;
constexpr float kDodgeDeadzone = 0.5f;

constexpr float kAirThrottleAccel = 200.f / 3.f;
constexpr float kGroundThrottleAccel = 1600.f;
constexpr float kThrottleDeadzone = 0.001f;
constexpr float kCoastBrake = 0.15f;
constexpr float kBoostPerSecond = kBoostMax / 3.f;
constexpr float kBoostMinTime = 0.1f;
constexpr float kBoostAccelGround = 2975.f / 3.f, kBoostAccelAir = 3175.f / 3.f;
constexpr float kSlideRise = 5.f, kSlideFall = 2.f;

constexpr float kTorqueScale = 2.f * kPi / 65536.f * 1000.f;
constexpr V3 kAirTorque{ 130.f, 95.f, 400.f };
constexpr V3 kAirDamping{ 30.f, 20.f, 50.f };
constexpr float kAutoflipImpulse = 200.f, kAutoflipTorque = 50.f, kAutoflipTime = 0.4f;
constexpr float kAutoflipNormZ = 0.70710678f, kAutoflipRoll = 2.8f;

constexpr float kCarCarFriction = 0.09f, kCarCarRestitution = 0.1f;
constexpr float kBumpCooldown = 0.25f, kBumpMinForward = 64.5f;
constexpr float kDemoRespawnTime = 3.f, kDemoInputDeadzone = 0.5f;
constexpr float kSupersonic = 2200.f;

constexpr float kBallMass = kCarMass / 6.f;
constexpr float kBallInvMass = 1.f / kBallMass;
constexpr float kBallMaxSpeed = 6000.f, kBallMaxAng = 6.f;
constexpr float kBallRestitution = 0.6f, kBallFriction = 0.35f;
constexpr float kBallInertia = 0.4f * kBallMass * kBallRadius * kBallRadius;
constexpr float kBallInvInertia = 1.f / kBallInertia;
// powf(1 - 0.03, 1/120) correctly rounded: per-tick ball drag in Bullet units
constexpr float kBallDrag = 0x1.ffdebcp-1f;

constexpr float kCarBallRestitution = 0.f, kCarBallFriction = 2.f, kCarBallBreak = 1.825f;
constexpr float kExtraZScale = 0.35f, kExtraFwdScale = 0.65f, kExtraMaxDv = 4600.f;

constexpr float kGoalCenterY = 5120.f, kGoalCenterZ = 321.3875f, kGoalThresholdY = 5124.25f;
constexpr float kBallArenaBreak = 1.905f;

constexpr float kSmallPadRadius = 144.f, kBigPadRadius = 208.f, kPadHeight = 95.f;
constexpr float kSmallPadAmount = 12.f, kBigPadAmount = 100.f;
constexpr float kSmallPadCooldown = 4.f, kBigPadCooldown = 10.f;

constexpr int kObsPerCar = 21;
constexpr int kStatePerCar = 22;
constexpr int kInternalFields = 19;

HDI constexpr int observationDim(int nCars, bool prev)
{
    return 9 + nCars * kObsPerCar + 2 * kPads + 6 + (nCars - 1) * 6 + 6 + 2 + 5 + (prev ? 8 : 0);
}
HDI constexpr int stateDim(int nCars) { return 9 + nCars * kStatePerCar + kPads; }

// wheel geometry
HDI V3 wheelAnchor(int w)
{
    const float x = w < 2 ? kFrontX : kBackX;
    const float ay = w < 2 ? kFrontY : kBackY;
    return V3{ x, (w & 1) ? -ay : ay, 0.f };
}
HDI float wheelRay(int w) { return w < 2 ? kFrontRay : kBackRay; }
HDI float wheelRadius(int w) { return w < 2 ? kFrontRadius : kBackRadius; }
HDI float wheelRest(int w) { return w < 2 ? kFrontRest : kBackRest; }
HDI float wheelScale(int w) { return w < 2 ? kSuspScaleFront : kSuspScaleBack; }

// Kickoff spawn order: index p in [0,120) excludes spawn p/24 and takes the
// (p%24)-th lexicographic permutation of the remaining four spawns.
HDI int kickoffSpawn(int perm, int slot)
{
    const int excluded = perm / 24;
    int r = perm % 24;
    int used = 0;  // bitmask over the 4 remaining spawns
    int result = 0;
    const int fact[4] = { 6, 2, 1, 1 };
    for (int p = 0; p <= slot; p++) {
        int q = r / fact[p];
        r %= fact[p];
        for (int j = 0; j < 4; j++) {
            if (used & (1 << j)) continue;
            if (q == 0) {
                used |= 1 << j;
                result = j < excluded ? j : j + 1;
                break;
            }
            q--;
        }
    }
    return result;
}

HDI float kickoffX(int i)
{
    return i == 0 ? -2048.f : (i == 1 ? 2048.f : (i == 2 ? -256.f : (i == 3 ? 256.f : 0.f)));
}
HDI float kickoffY(int i) { return i < 2 ? -2560.f : (i < 4 ? -3840.f : -4608.f); }
HDI float kickoffYaw(int i) { return i == 0 ? kPi4 * 1 : (i == 1 ? kPi4 * 3 : kPi4 * 2); }
HDI float respawnX(int i) { return i == 0 ? 2688.f : (i == 1 ? 2304.f : (i == 2 ? -2304.f : -2688.f)); }
constexpr float kRespawnY = -4608.f;
constexpr float kRespawnYaw = kPi2 * 1;

// boost pad positions (x, y, z) - big pads first
static __device__ __constant__ const float kPadPos[kPads][3] = {
    { -3584.f, 0.f, 73.f }, { 3584.f, 0.f, 73.f }, { -3072.f, 4096.f, 73.f }, { 3072.f, 4096.f, 73.f },
    { -3072.f, -4096.f, 73.f }, { 3072.f, -4096.f, 73.f },
    { 0.f, -4240.f, 70.f }, { -1792.f, -4184.f, 70.f }, { 1792.f, -4184.f, 70.f }, { -940.f, -3308.f, 70.f },
    { 940.f, -3308.f, 70.f }, { 0.f, -2816.f, 70.f }, { -3584.f, -2484.f, 70.f }, { 3584.f, -2484.f, 70.f },
    { -1788.f, -2300.f, 70.f }, { 1788.f, -2300.f, 70.f }, { -2048.f, -1036.f, 70.f }, { 0.f, -1024.f, 70.f },
    { 2048.f, -1036.f, 70.f }, { -1024.f, 0.f, 70.f }, { 1024.f, 0.f, 70.f }, { -2048.f, 1036.f, 70.f },
    { 0.f, 1024.f, 70.f }, { 2048.f, 1036.f, 70.f }, { -1788.f, 2300.f, 70.f }, { 1788.f, 2300.f, 70.f },
    { -3584.f, 2484.f, 70.f }, { 3584.f, 2484.f, 70.f }, { 0.f, 2816.f, 70.f }, { -940.f, 3308.f, 70.f },
    { 940.f, 3308.f, 70.f }, { -1792.f, 4184.f, 70.f }, { 1792.f, 4184.f, 70.f }, { 0.f, 4240.f, 70.f },
};

// Pad seen by an orange observer at slot p: the pad mirrored through the
// field centre, (x, y) -> (-x, -y).
HDI int mirroredPad(int p)
{
    if (p >= 6) return 39 - p;
    return p < 2 ? 1 - p : 7 - p;
}

}  // namespace carl
