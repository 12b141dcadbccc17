// car_phase.h - per-car device physics of one tick.
//
// Reference semantics, per stage of RLEnvironment::step
// (src/RLEnvironment.cu:166-211):
//   broadphase             include/Physics/CarArena/BroadPhase.cuh:10-28
//   suspension raycast     include/Physics/SuspensionRaycast.cuh:25-301
//   controls               include/Physics/Controls.cuh, Controls/{Context,Drive,Aerial}.cuh
//   box-triangle SAT       include/Physics/CarArena/SAT.cuh:42-161
//   clip / contacts        include/Physics/CarArena/Clip.cuh:53-377
//   manifold               include/Physics/CarArena/Manifold.cuh:73-310
//   suspension forces      include/Physics/CarSuspension.cuh:8-339
//   contact solver         include/Physics/CarArena/Solve.cuh:42-314
//   integration            include/Physics/Integration.cuh:6-69
//
// Structure differs from the reference: SAT, clipping and best-contact
// selection are one streaming pass over the car's grid cell (no pair /
// contact buffers in memory), and hits are taken in cell-list order (the
// reference's atomicAdd slot order is nondeterministic).
#pragma once

#include "state.h"

namespace carl {

// ---------------------------------------------------------------- kinematics

DI Q4 integrateRotation(Q4 rot, V3 ang)
{
    constexpr float dt = kDt;
    constexpr float maxMotion = kAngMotionThresh;
    const float speedSq = lensq(ang);
    float speed = speedSq > 1e-8f ? sqrtf(speedSq) : 0.f;
    if (speed * dt > maxMotion) speed = maxMotion / dt;
    float s, c;
    sincos_(0.5f * speed * dt, &s, &c);
    V3 axis;
    if (speed < 0.001f) {
        // Taylor expansion of sin(x/2)/x for tiny rotations
        const float dtSq = dt * dt;
        const float scale = 0.5f * dt - dtSq * dt * 0.020833333333f * speed * speed;
        axis = ang * scale;
    } else {
        axis = ang * (s / speed);
    }
    const Q4 delta{ axis.x, axis.y, axis.z, c };
    const Q4 basis = quatFromColumns(rotate(rot, kX), rotate(rot, kY), rotate(rot, kZ));
    return qnormalize(qmul(delta, basis));
}

DI void integratePose(V3& pos, V3& cen, Q4& rot, V3 vel, V3 ang)
{
    pos = pos + vel * kDt;
    rot = integrateRotation(rot, ang);
    cen = pos + rotate(rot, kHitboxOffset);
}

DI V3 boxAabbMin(V3 cen, Q4 rot)
{
    const V3 rx = rotate(rot, kX), ry = rotate(rot, kY), rz = rotate(rot, kZ);
    const V3 half = (vabs(rx) * kHalf.x + vabs(ry) * kHalf.y) + vabs(rz) * kHalf.z;
    return cen - half;
}

struct Broad {
    int start;
    int count;
    int cell;   // the cell's coordinates, x | y << 6 | z << 12
};

// grid cell of the min corner of the swept (current + predicted) AABB
DI Broad broadphase(const Dev& d, V3 pos, V3 vel, V3 ang, V3 cen, Q4 rot)
{
    V3 ppos = pos, pcen;
    Q4 prot = rot;
    integratePose(ppos, pcen, prot, vel, ang);
    const V3 swept = vmin(boxAabbMin(cen, rot), boxAabbMin(pcen, prot));
    int cx, cy, cz;
    cellOf(swept, cx, cy, cz);
    const int cell = flatCell(cx, cy, cz);
    const int s = d.arena.cellStart[cell];
    return Broad{ s, d.arena.cellStart[cell + 1] - s, cx | cy << 6 | cz << 12 };
}

// ------------------------------------------------------------------ raycast

struct Wheels {
    float dist[kWheels];
    V3 normal[kWheels];
    int src[kWheels];
};

DI V3 wheelStart(V3 cen, Q4 rot, int w) { return cen + rotate(rot, wheelAnchor(w)); }

DI bool raySphere(V3 start, V3 dir, V3 center, float radius, float maxDist, float& dist)
{
    const V3 off = start - center;
    const float b = dot(off, dir);
    const float c = lensq(off) - radius * radius;
    if (c < 0.f) return false;
    const float disc = b * b - c;
    if (disc < 0.f) return false;
    dist = -b - sqrtf(disc);
    return dist > 0.f && dist <= maxDist;
}

DI bool rayBox(V3 start, V3 dir, V3 center, Q4 rot, float maxDist, float& dist, V3& normal)
{
    const V3 ls = unrotate(rot, start - center);
    const V3 ld = unrotate(rot, dir);
    float entry = 0.f, exitD = maxDist;
    int hitAxis = -1;
#pragma unroll
    for (int a = 0; a < 3; a++) {
        const float dd = comp(ld, a), s = comp(ls, a), h = comp(kHalf, a);
        if (fabsf(dd) < 1e-8f) {
            if (fabsf(s) > h) return false;
            continue;
        }
        const float inv = 1.f / dd;
        const float t1 = (-h - s) * inv;
        const float t2 = (h - s) * inv;
        const float tn = fmin_(t1, t2);
        if (tn > entry) { entry = tn; hitAxis = a; }
        exitD = fmin_(exitD, fmax_(t1, t2));
        if (entry > exitD) return false;
    }
    if (hitAxis < 0) return false;
    dist = entry;
    V3 ln = kZero;
    setComp(ln, hitAxis, comp(ld, hitAxis) > 0.f ? -1.f : 1.f);
    normal = rotate(rot, ln);
    return true;
}

// Every wheel ray ends within kWheelReach of the car's box centre: the
// anchors lie at most 56.1 uu from it, and a ray is at most the longer of the
// two ray lengths; 4 uu spare cover the rounding of the rays' arithmetic.  A
// body whose centre is farther than kWheelReach plus its bounding radius
// meets no wheel ray, so its rays are not cast (each would miss).
constexpr float kWheelReach = 56.1f + (kFrontRay > kBackRay ? kFrontRay : kBackRay) + 4.f;
constexpr float kCarRayReach = kWheelReach + 80.f;   // + |kHalf| (76.6) rounded up
constexpr float kBallRayReach = kWheelReach + kBallRadius;

// rays against the other cars of the simulation, then the ball (after the
// arena, so only strictly nearer hits replace an arena hit)
// the wheel rays against one other car's box
DI void raycastCar(const V3* start, V3 dir, V3 ocen, Q4 orot, Wheels& w)
{
#pragma unroll
    for (int k = 0; k < kWheels; k++) {
        float dd;
        V3 n;
        if (!rayBox(start[k], dir, ocen, orot, wheelRay(k), dd, n) || dd >= w.dist[k]) continue;
        w.dist[k] = dd;
        w.normal[k] = n;
        w.src[k] = kSrcCar;
    }
}

// the wheel rays against the ball
DI void raycastBall(const V3* start, V3 dir, V3 ball, Wheels& w)
{
    const float invR = 1.f / kBallRadius;
#pragma unroll
    for (int k = 0; k < kWheels; k++) {
        float dd;
        if (!raySphere(start[k], dir, ball, kBallRadius, wheelRay(k), dd) || dd >= w.dist[k]) continue;
        w.dist[k] = dd;
        w.normal[k] = ((start[k] + dir * dd) - ball) * invR;
        w.src[k] = kSrcBall;
    }
}

// the wheel rays against the simulation's other cars, in car order, then the ball
DI void raycastBodies(const Dev& d, int car, int sim, V3 cen, const V3* start, V3 dir, Wheels& w)
{
    const int base = sim * d.nCars;
    const V3 ball = d.sv(CARL_SIM_BALL_POS, sim);
    for (int o = 0; o < d.nCars; o++) {
        const int oc = base + o;
        // the other car's words are loaded together, before its demolished
        // flag is tested (one round trip instead of two)
        const int demoed = d.ci(CARL_CAR_DEMOED, oc);
        const V3 ocen = d.cv(CARL_CAR_CEN, oc);
        const Q4 orot = d.cq(CARL_CAR_ROT, oc);
        if (oc == car || demoed || lensq(ocen - cen) > kCarRayReach * kCarRayReach) continue;
        raycastCar(start, dir, ocen, orot, w);
    }
    if (!(lensq(ball - cen) > kBallRayReach * kBallRayReach)) raycastBall(start, dir, ball, w);
}

DI void storeWheelOutputs(const Dev& d, int car, const Wheels& w)
{
#pragma unroll
    for (int k = 0; k < kWheels; k++) {
        d.seti(CARL_CAR_WHEEL_SOURCE + k, car, w.src[k]);
        d.seti(CARL_CAR_WHEEL_CONTACT + k, car, (w.src[k] != kSrcNone && w.dist[k] <= wheelRay(k)) ? 1 : 0);
    }
}

// ------------------------------------------------------------------ controls

struct Controls {
    float throttle, steer, yaw, pitch, roll;
    int jump, boost, slide;
};

// include/State/Controls.cuh:57-112 (steer and yaw share the horizontal axis)
DI Controls decodeControls(int kind, const void* actions, int car)
{
    Controls c;
    if (kind == CARL_ACTIONS_DISCRETE) {
        const int32_t* a = (const int32_t*)actions + 7 * car;
        auto axis = [](int32_t v) { return v == 1 ? -1.f : (v == 2 ? 1.f : 0.f); };
        const float h = axis(a[0]);
        c.throttle = axis(a[2]); c.steer = h; c.yaw = h;
        c.pitch = axis(a[1]); c.roll = axis(a[5]);
        c.jump = a[6] == 1; c.boost = a[4] == 1; c.slide = a[3] == 1;
    } else if (kind == CARL_ACTIONS_CONTINUOUS) {
        const float* a = (const float*)actions + 7 * car;
        auto axis = [](float v) { return v < -1.f ? -1.f : (v > 1.f ? 1.f : v); };
        const float h = axis(a[0]);
        c.throttle = axis(a[2]); c.steer = h; c.yaw = h;
        c.pitch = axis(a[1]); c.roll = axis(a[5]);
        c.jump = a[6] >= .5f; c.boost = a[4] >= .5f; c.slide = a[3] >= .5f;
    } else {
        const carl_controls a = ((const carl_controls*)actions)[car];
        c.throttle = a.throttle; c.steer = a.steer; c.yaw = a.yaw; c.pitch = a.pitch; c.roll = a.roll;
        c.jump = a.jump; c.boost = a.boost; c.slide = a.slide;
    }
    return c;
}

// register copy of the car fields the arena phase reads and writes
struct CarRegs {
    V3 pos, vel, ang, cen;
    Q4 rot;
    int onGround;
    float airTime, airTimeSinceJump, handbrake;
    int hasJumped, isJumping;
    float jumpTime;
    int lastJump, hasDoubleJumped, hasFlipped, isFlipping;
    float flipTime;
    int isAutoFlipping;
    float autoFlipTimer, autoFlipScale;
    V3 flipTorque;
    int isBoosting;
    float boost, boostingTime, timeSinceBoosted;
    float brake, steer, drive;                    // staged for the next tick
    float brakePrev, steerPrev, drivePrev;        // consumed this tick
    float throttleVal, rawThrottle, handbrakeVal;
    V3 jumpImp, angImp;
    float latF[kWheels], lonF[kWheels];
    int manCount;
    V3 manNormal;
};

DI void loadRegs(const Dev& d, int c, CarRegs& r)
{
    r.pos = d.cv(CARL_CAR_POS, c); r.vel = d.cv(CARL_CAR_VEL, c); r.ang = d.cv(CARL_CAR_ANG, c);
    r.cen = d.cv(CARL_CAR_CEN, c); r.rot = d.cq(CARL_CAR_ROT, c);
    r.onGround = d.ci(CARL_CAR_ON_GROUND, c);
    r.airTime = d.cf(CARL_CAR_AIR_TIME, c);
    r.airTimeSinceJump = d.cf(CARL_CAR_AIR_TIME_SINCE_JUMP, c);
    r.handbrake = d.cf(CARL_CAR_HANDBRAKE, c);
    r.hasJumped = d.ci(CARL_CAR_HAS_JUMPED, c);
    r.isJumping = d.ci(CARL_CAR_IS_JUMPING, c);
    r.jumpTime = d.cf(CARL_CAR_JUMP_TIME, c);
    r.lastJump = d.ci(CARL_CAR_LAST_JUMP, c);
    r.hasDoubleJumped = d.ci(CARL_CAR_HAS_DOUBLE_JUMPED, c);
    r.hasFlipped = d.ci(CARL_CAR_HAS_FLIPPED, c);
    r.isFlipping = d.ci(CARL_CAR_IS_FLIPPING, c);
    r.flipTime = d.cf(CARL_CAR_FLIP_TIME, c);
    r.isAutoFlipping = d.ci(CARL_CAR_IS_AUTO_FLIPPING, c);
    r.autoFlipTimer = d.cf(CARL_CAR_AUTO_FLIP_TIMER, c);
    r.autoFlipScale = d.cf(CARL_CAR_AUTO_FLIP_SCALE, c);
    r.flipTorque = d.cv(CARL_CAR_FLIP_TORQUE, c);
    r.isBoosting = d.ci(CARL_CAR_IS_BOOSTING, c);
    r.boost = d.cf(CARL_CAR_BOOST, c);
    r.boostingTime = d.cf(CARL_CAR_BOOSTING_TIME, c);
    r.timeSinceBoosted = d.cf(CARL_CAR_TIME_SINCE_BOOSTED, c);
    r.brake = d.cf(CARL_CAR_BRAKE_STAGE, c);
    r.steer = d.cf(CARL_CAR_STEER_STAGE, c);
    r.drive = d.cf(CARL_CAR_DRIVE_STAGE, c);
    r.brakePrev = r.steerPrev = r.drivePrev = 0.f;
    r.throttleVal = r.rawThrottle = r.handbrakeVal = 0.f;
    r.jumpImp = kZero;
    r.angImp = kZero;
#pragma unroll
    for (int k = 0; k < kWheels; k++) {
        r.latF[k] = d.cf(CARL_CAR_LAT_FRICTION + k, c);
        r.lonF[k] = d.cf(CARL_CAR_LON_FRICTION + k, c);
    }
    r.manCount = d.ci(CARL_CAR_MANIFOLD_COUNT, c);
    r.manNormal = d.cv(CARL_CAR_MANIFOLD_NORMAL, c);
}

DI void storeRegs(const Dev& d, int c, const CarRegs& r)
{
    d.setv(CARL_CAR_POS, c, r.pos); d.setv(CARL_CAR_VEL, c, r.vel); d.setv(CARL_CAR_ANG, c, r.ang);
    d.setv(CARL_CAR_CEN, c, r.cen); d.setq(CARL_CAR_ROT, c, r.rot);
    d.seti(CARL_CAR_ON_GROUND, c, r.onGround);
    d.setf(CARL_CAR_AIR_TIME, c, r.airTime);
    d.setf(CARL_CAR_AIR_TIME_SINCE_JUMP, c, r.airTimeSinceJump);
    d.setf(CARL_CAR_HANDBRAKE, c, r.handbrake);
    d.seti(CARL_CAR_HAS_JUMPED, c, r.hasJumped);
    d.seti(CARL_CAR_IS_JUMPING, c, r.isJumping);
    d.setf(CARL_CAR_JUMP_TIME, c, r.jumpTime);
    d.seti(CARL_CAR_LAST_JUMP, c, r.lastJump);
    d.seti(CARL_CAR_HAS_DOUBLE_JUMPED, c, r.hasDoubleJumped);
    d.seti(CARL_CAR_HAS_FLIPPED, c, r.hasFlipped);
    d.seti(CARL_CAR_IS_FLIPPING, c, r.isFlipping);
    d.setf(CARL_CAR_FLIP_TIME, c, r.flipTime);
    d.seti(CARL_CAR_IS_AUTO_FLIPPING, c, r.isAutoFlipping);
    d.setf(CARL_CAR_AUTO_FLIP_TIMER, c, r.autoFlipTimer);
    d.setf(CARL_CAR_AUTO_FLIP_SCALE, c, r.autoFlipScale);
    d.setv(CARL_CAR_FLIP_TORQUE, c, r.flipTorque);
    d.seti(CARL_CAR_IS_BOOSTING, c, r.isBoosting);
    d.setf(CARL_CAR_BOOST, c, r.boost);
    d.setf(CARL_CAR_BOOSTING_TIME, c, r.boostingTime);
    d.setf(CARL_CAR_TIME_SINCE_BOOSTED, c, r.timeSinceBoosted);
    d.setf(CARL_CAR_BRAKE_STAGE, c, r.brake);
    d.setf(CARL_CAR_STEER_STAGE, c, r.steer);
    d.setf(CARL_CAR_DRIVE_STAGE, c, r.drive);
#pragma unroll
    for (int k = 0; k < kWheels; k++) {
        d.setf(CARL_CAR_LAT_FRICTION + k, c, r.latF[k]);
        d.setf(CARL_CAR_LON_FRICTION + k, c, r.lonF[k]);
    }
    d.seti(CARL_CAR_MANIFOLD_COUNT, c, r.manCount);
    d.setv(CARL_CAR_MANIFOLD_NORMAL, c, r.manNormal);
}

DI float steerCurve(float x)
{
    if (x <= 0.f) return 0.53356f;
    if (x <= 500.f) return 0.53356f + (0.31930f - 0.53356f) * (x / 500.f);
    if (x <= 1000.f) return 0.31930f + (0.18203f - 0.31930f) * ((x - 500.f) / 500.f);
    if (x <= 1500.f) return 0.18203f + (0.10570f - 0.18203f) * ((x - 1000.f) / 500.f);
    if (x <= 1750.f) return 0.10570f + (0.08507f - 0.10570f) * ((x - 1500.f) / 250.f);
    if (x <= 3000.f) return 0.08507f + (0.03454f - 0.08507f) * ((x - 1750.f) / 1250.f);
    return 0.03454f;
}

DI float slideSteerCurve(float x)
{
    if (x <= 0.f) return 0.39235f;
    if (x <= 2500.f) return 0.39235f + (0.12610f - 0.39235f) * (x / 2500.f);
    return 0.12610f;
}

DI float driveTorqueCurve(float x)
{
    if (x <= 0.f) return 1.f;
    if (x >= 1410.f) return 0.f;
    if (x <= 1400.f) return 1.f - (x / 1400.f) * 0.9f;
    return 0.1f * (1.f - (x - 1400.f) / 10.f);
}

struct Frame {
    Q4 rot;
    V3 fwd, up;
    float fwdSpeed, absFwdSpeed;
    int wheelCount;
    bool onGround, jumpPressed;
};

// flip start: normalized dodge direction -> torque axis and impulse
DI void startFlip(CarRegs& r, const Frame& f, V3 dodge)
{
    r.flipTime = 0.f;
    r.hasFlipped = 1;
    r.isFlipping = 1;
    if (fabsf(dodge.x) < 0.1f && fabsf(dodge.y) < 0.1f) dodge = kZero;
    else dodge = dodge * rsqrt_(lensq(dodge));
    r.flipTorque = V3{ -dodge.y, dodge.x, 0.f };

    V3 dd = dodge;
    if (fabsf(dd.x) < 0.1f) dd.x = 0.f;
    if (fabsf(dd.y) < 0.1f) dd.y = 0.f;
    const float speedScale = clamp_(f.absFwdSpeed / kCarMaxSpeed, 0.f, 1.f);
    const bool backward = f.absFwdSpeed < 100.f ? dd.x < 0.f : ((dd.x >= 0.f) != (f.fwdSpeed >= 0.f));
    const float maxFwd = backward ? kFlipBackScale : kFlipFwdScale;
    V3 lv = dd * kFlipInitialVel;
    lv.x *= (maxFwd - 1.f) * speedScale + 1.f;
    lv.y *= (kFlipSideScale - 1.f) * speedScale + 1.f;
    if (backward) lv.x *= kFlipBackX;

    const V3 flat{ f.fwd.x, f.fwd.y, 0.f };
    const float den = lensq(flat);
    const V3 flatN = den > 1e-12f ? flat * rsqrt_(den) : kX;
    const V3 right{ -flatN.y, flatN.x, 0.f };
    r.vel = r.vel + (flatN * lv.x + right * lv.y);
}

DI void applyControls(CarRegs& r, const Controls& c, const Wheels& w)
{
    Frame f;
    f.rot = r.rot;
    f.fwd = rotate(r.rot, kX);
    f.up = rotate(r.rot, kZ);
    f.fwdSpeed = dot(r.vel, f.fwd);
    f.absFwdSpeed = fabsf(f.fwdSpeed);
    int n = 0;
#pragma unroll
    for (int k = 0; k < kWheels; k++) n += w.dist[k] <= wheelRay(k) ? 1 : 0;
    f.wheelCount = n;
    f.onGround = n >= 3;
    f.jumpPressed = c.jump && !r.lastJump;
    r.lastJump = c.jump;
    r.onGround = f.onGround;

    // ground drive, staged one tick late (Drive.cuh:42-93)
    {
        const float throttle = (c.boost && r.boost > 0.f) ? 1.f : c.throttle;
        const bool opposing = f.absFwdSpeed > kStoppingVel && ((throttle > 0.f) != (f.fwdSpeed > 0.f));
        float brake;
        if (f.wheelCount == 0 || c.slide) brake = 0.f;
        else if (fabsf(throttle) >= kThrottleDeadzone) brake = opposing ? 1.f : 0.f;
        else brake = f.absFwdSpeed < kStoppingVel ? 1.f : kCoastBrake;
        float drive;
        if (f.wheelCount == 0 || fabsf(throttle) < kThrottleDeadzone || (!c.slide && opposing)) {
            drive = 0.f;
        } else {
            float scale = driveTorqueCurve(f.absFwdSpeed);
            if (f.wheelCount < 3) scale *= 0.25f;
            drive = throttle * kGroundThrottleAccel * scale;
        }
        r.brakePrev = r.brake; r.brake = brake;
        r.throttleVal = throttle;
        r.rawThrottle = c.throttle;
        r.drivePrev = r.drive; r.drive = drive;
    }

    // boost (Drive.cuh:95-121)
    {
        bool boosting;
        if (r.boost <= 0.f) boosting = false;
        else if (!r.isBoosting) boosting = c.boost != 0;
        else boosting = c.boost || r.boostingTime < kBoostMinTime;
        r.isBoosting = boosting;
        if (boosting) {
            r.boostingTime += kDt;
            r.boost = fmax_(r.boost - kBoostPerSecond * kDt, 0.f);
            const float accel = f.onGround ? kBoostAccelGround : kBoostAccelAir;
            r.jumpImp = r.jumpImp + f.fwd * (accel * kDt);
            r.timeSinceBoosted = 0.f;
        } else {
            r.boostingTime = 0.f;
            r.timeSinceBoosted += kDt;
        }
        r.boost = fmin_(r.boost, kBoostMax);
    }

    // steer (Drive.cuh:123-146)
    {
        if (c.slide) r.handbrake += kSlideRise * kDt;
        else r.handbrake -= kSlideFall * kDt;
        r.handbrake = clamp_(r.handbrake, 0.f, 1.f);
        r.handbrakeVal = r.handbrake;
        float angle = steerCurve(f.absFwdSpeed);
        if (r.handbrake > 0.f) {
            const float sl = slideSteerCurve(f.absFwdSpeed);
            angle += (sl - angle) * r.handbrake;
        }
        r.steerPrev = r.steer;
        r.steer = angle * c.steer;
    }

    // air control with fewer than three wheels in contact (Aerial.cuh:244-342)
    if (f.wheelCount < 3) {
        bool useAir = true;
        if (r.isFlipping) r.isFlipping = r.hasFlipped && r.flipTime < kFlipTorqueTime;
        if (r.isFlipping && lensq(r.flipTorque) > 1e-12f) {
            const V3 rel = r.flipTorque;
            float pitchScale = 1.f;
            useAir = false;
            if ((rel.y != 0.f && c.pitch != 0.f) && ((rel.y > 0.f) == (c.pitch > 0.f))) {
                pitchScale = 1.f - fmin_(fabsf(c.pitch), 1.f);
                useAir = true;
            }
            const V3 relTorque{ rel.x * kFlipTorqueX, rel.y * kFlipTorqueY * pitchScale, 0.f };
            r.angImp = r.angImp + rotate(f.rot, relTorque) * kDt;
        }
        if (useAir && f.wheelCount == 0 && !r.isAutoFlipping) {
            const bool locked = r.isFlipping || (r.hasFlipped && r.flipTime < kFlipTorqueTime + kFlipPitchlockExtra);
            const float pitchScale = locked ? 0.f : 1.f;
            const V3 input{ c.pitch, c.yaw, c.roll };
            const V3 ctlScale{ pitchScale, 1.f, 1.f };
            const V3 dampIn{ c.pitch * pitchScale, c.yaw, 0.f };
            V3 torque = kZero, damping = kZero;
            const bool hasInput = lensq(input) > 0.f;
#pragma unroll
            for (int i = 0; i < 3; i++) {
                const V3 dir = i == 0 ? -rotate(f.rot, kY) : (i == 1 ? f.up : -f.fwd);
                const float control = comp(input, i) * comp(ctlScale, i);
                const float proj = dot(dir, r.ang);
                const float damp = proj * comp(kAirDamping, i) * (1.f - fabsf(comp(dampIn, i)));
                if (hasInput) torque = torque + dir * (control * comp(kAirTorque, i));
                damping = damping + dir * damp;
            }
            r.angImp = r.angImp + (torque - damping) * (kTorqueScale * kDt);
        }
        if (c.throttle != 0.f) r.jumpImp = r.jumpImp + f.fwd * (c.throttle * kAirThrottleAccel * kDt);
    }

    // jump (Aerial.cuh:15-73)
    {
        const bool grace = r.hasJumped && r.jumpTime < kJumpMinTime + kJumpResetPad;
        if (f.onGround && !r.isJumping && !grace) { r.hasJumped = 0; r.jumpTime = 0.f; }
        if (r.isJumping) {
            r.isJumping = (r.jumpTime < kJumpMinTime || (c.jump && r.jumpTime < kJumpMaxTime)) ? 1 : 0;
        } else if (f.onGround && f.jumpPressed) {
            r.isJumping = 1;
            r.jumpTime = 0.f;
            r.jumpImp = r.jumpImp + f.up * kJumpImmediate;
        }
        if (r.isJumping) {
            r.hasJumped = 1;
            float accel = kJumpAccel;
            if (r.jumpTime < kJumpMinTime) accel *= 0.62f;
            r.jumpImp = r.jumpImp + f.up * (accel * kDt);
        }
        if (r.isJumping || r.hasJumped) r.jumpTime += kDt;
    }

    // auto-flip against an upward facing contact of the previous tick (Drive.cuh:134-178)
    {
        if (f.jumpPressed && r.manCount != 0 && r.manNormal.z > kAutoflipNormZ) {
            const V3 right = rotate(f.rot, kY);
            const float roll = -atan2_(right.z, f.up.z);
            const float absRoll = fabsf(roll);
            if (absRoll > kAutoflipRoll) {
                r.autoFlipTimer = kAutoflipTime * (absRoll / kPi);
                r.autoFlipScale = roll > 0.f ? 1.f : -1.f;
                r.isAutoFlipping = 1;
                r.vel = r.vel + f.up * -kAutoflipImpulse;
            }
        }
        if (r.isAutoFlipping) {
            if (r.autoFlipTimer <= 0.f) {
                r.isAutoFlipping = 0;
                r.autoFlipTimer = 0.f;
            } else {
                const float torque = kAutoflipTorque * r.autoFlipScale * kDt;
                r.ang = r.ang + f.fwd * torque;
                r.autoFlipTimer -= kDt;
            }
        }
    }

    // dodge / double jump and flip motion (Aerial.cuh:120-235)
    {
        if (f.onGround) {
            r.hasDoubleJumped = 0; r.hasFlipped = 0; r.isFlipping = 0;
            r.airTime = 0.f; r.airTimeSinceJump = 0.f; r.flipTime = 0.f;
        } else {
            r.airTime += kDt;
            if (r.hasJumped && !r.isJumping) r.airTimeSinceJump += kDt;
            else r.airTimeSinceJump = 0.f;
            const bool canDodge = !r.hasFlipped && !r.hasDoubleJumped && r.airTimeSinceJump < kDoubleJumpWindow;
            if (f.jumpPressed && canDodge) {
                const V3 dodge{ -c.pitch, c.yaw + c.roll, 0.f };
                const float mag = fabsf(c.yaw) + fabsf(c.pitch) + fabsf(c.roll);
                if (mag >= kDodgeDeadzone) {
                    startFlip(r, f, dodge);
                } else {
                    r.vel = r.vel + f.up * kJumpImmediate;
                    r.hasDoubleJumped = 1;
                }
            }
        }
        if (!r.isFlipping) {
            if (r.hasFlipped) r.flipTime += kDt;
        } else {
            r.flipTime += kDt;
            if (r.flipTime <= kFlipTorqueTime) {
                const bool dampZ = r.flipTime >= kFlipZDampStart && (r.vel.z < 0.f || r.flipTime < kFlipZDampEnd);
                if (dampZ) r.vel.z *= 1.f - kFlipZDamp;
            }
        }
    }
}

// ------------------------------------------------------- car vs arena mesh

struct LocalTri {
    V3 v0, v1, v2, e0, e1, e2, delta;
};

DI LocalTri toLocal(const Tri& t, V3 cen, Q4 rot)
{
    LocalTri l;
    l.v0 = unrotate(rot, t.v0 - cen);
    l.v1 = unrotate(rot, t.v1 - cen);
    l.v2 = unrotate(rot, t.v2 - cen);
    l.e0 = l.v1 - l.v0;
    l.e1 = l.v2 - l.v1;
    l.e2 = l.v0 - l.v2;
    l.delta = -(((l.v0 + l.v1) + l.v2) / 3.f);
    return l;
}

DI V3 triVert(const LocalTri& t, int i) { return sel(i == 0, t.v0, sel(i == 1, t.v1, t.v2)); }
DI V3 triEdge(const LocalTri& t, int i) { return sel(i == 0, t.e0, sel(i == 1, t.e1, t.e2)); }

struct Sat {
    bool overlap;
    int axisIdx;
    float minPen;
    V3 minAxis;
};

DI void satAxis(V3 ax, const LocalTri& t, int idx, bool norm, Sat& s)
{
    if (!s.overlap) return;
    const float l = lensq(ax);
    if (l < 1e-12f) return;
    if (norm) ax = ax * rsqrt_(l);
    ax = ax * copysignf(1.f, dot(ax, t.delta));
    const float rr = dot(vabs(ax), kHalf);
    const float d0 = dot(t.v0, ax), d1 = dot(t.v1, ax), d2 = dot(t.v2, ax);
    const float tMin = fmin_(fmin_(d0, d1), d2);
    const float tMax = fmax_(fmax_(d0, d1), d2);
    if (rr < tMin || tMax < -rr) { s.overlap = false; return; }
    const float depth = fmin_(rr - tMin, tMax - -rr);
    if (depth < s.minPen) { s.minPen = depth; s.minAxis = ax; s.axisIdx = idx; }
}

DI Sat boxTriSat(const LocalTri& t)
{
    // The box face axes first, as a pure rejection: the overlap verdict is the
    // conjunction over all axes, so testing three of them early changes
    // nothing, and they are cheap (no normalisation); most cell triangles
    // miss the box along one of them.  The bookkeeping pass below then runs
    // every axis in the reference order.
    Sat pre{ true, 0, kFltMax, kZero };
    satAxis(kX, t, 1, false, pre);
    satAxis(kY, t, 2, false, pre);
    satAxis(kZ, t, 3, false, pre);
    if (!pre.overlap) return pre;
    Sat s{ true, 0, kFltMax, kZero };
    satAxis(cross(t.e0, t.e1), t, 0, true, s);
    if (!s.overlap) return s;
    satAxis(kX, t, 1, false, s);
    satAxis(kY, t, 2, false, s);
    satAxis(kZ, t, 3, false, s);
#pragma unroll
    for (int a = 0; a < 3; a++) {
#pragma unroll
        for (int e = 0; e < 3; e++) satAxis(cross(triEdge(t, e), unitAxis(a)), t, 4 + 3 * a + e, true, s);
    }
    return s;
}

struct Contact {
    V3 carPos, arenaPos, normal;
    float depth;
};

// Sutherland-Hodgman against one plane; output capped at kMaxPolygon vertices
// (only reachable through rounding on near-degenerate polygons).  The polygon
// lives in registers: every slot access is unrolled, writes select their slot.
constexpr int kMaxPolygon = 8;

struct Poly {
    V3 v[kMaxPolygon];
    int n;
};

DI void polyPut(Poly& p, V3 x)
{
    setAt(p.v, p.n, x);
    p.n++;
}

DI Poly clipPolygon(const Poly& in, V3 normal, float dist)
{
    Poly out;
#pragma unroll
    for (int j = 0; j < kMaxPolygon; j++) out.v[j] = kZero;
    out.n = 0;
#pragma unroll
    for (int i = 0; i < kMaxPolygon; i++) {
        if (i >= in.n) break;
        const V3 cur = in.v[i];
        V3 nxt = in.v[0];
        if (i + 1 < kMaxPolygon && i + 1 < in.n) nxt = in.v[i + 1 < kMaxPolygon ? i + 1 : 0];
        const float cd = dot(normal, cur) - dist;
        const float nd = dot(normal, nxt) - dist;
        const bool ci = cd <= 0.f, ni = nd <= 0.f;
        if (ci && out.n < kMaxPolygon) polyPut(out, cur);
        if (ci != ni && out.n < kMaxPolygon) {
            const float t = cd / (cd - nd);
            polyPut(out, cur + (nxt - cur) * t);
        }
    }
    return out;
}

DI Contact edgeContact(const LocalTri& t, float minPen, int axisIdx, V3 sep)
{
    const int carAxis = (axisIdx - 4) / 3;
    const int triEdgeIdx = (axisIdx - 4) % 3;
    const V3 center = ((t.v0 + t.v1) + t.v2) / 3.f;
    if (dot(sep, center) > 0.f) sep = -sep;
    V3 carPoint = vsign(-sep) * kHalf;
    setComp(carPoint, carAxis, 0.f);
    const V3 carAx = unitAxis(carAxis);
    const V3 triPoint = triVert(t, triEdgeIdx);
    const V3 edge = triEdge(t, triEdgeIdx);
    const float triLen = len(edge);
    const V3 triAx = edge / triLen;
    const V3 carToTri = triPoint - carPoint;
    const float ad = dot(carAx, triAx);
    const float den = 1.f - ad * ad;
    V3 onTri = triPoint;
    if (den > 1e-6f) {
        const float carProj = dot(carToTri, carAx);
        const float triProj = dot(carToTri, triAx);
        const float un = (ad * carProj - triProj) / den;
        onTri = triPoint + triAx * clamp_(un, 0.f, triLen);
    }
    const float h = comp(kHalf, carAxis);
    const float cp = clamp_(dot(carAx, onTri - carPoint), -h, h);
    const V3 onCar = carPoint + carAx * cp;
    const V3 sv = onTri - onCar;
    const float sq = lensq(sv);
    Contact r{ onCar, onTri, sep, minPen };
    if (sq > 1e-8f) {
        V3 nn = sv * rsqrt_(sq);
        if (dot(nn, center) > 0.f) nn = -nn;
        r.normal = nn;
    }
    return r;
}

struct ManPt {
    V3 carPos, worldPos, worldNormal;
    float dist;
};

DI ManPt sel(bool c, const ManPt& a, const ManPt& b)
{
    return ManPt{ sel(c, a.carPos, b.carPos), sel(c, a.worldPos, b.worldPos), sel(c, a.worldNormal, b.worldNormal),
                  sel(c, a.dist, b.dist) };
}

constexpr float kManifoldBreakSq = kContactBreak * kContactBreak;

DI bool nearManifold(const ManPt* pts, int n, V3 carPos)
{
    bool near = false;
#pragma unroll
    for (int i = 0; i < kMaxManifold; i++)
        if (i < n && lensq(pts[i].carPos - carPos) < kManifoldBreakSq) near = true;
    return near;
}

DI int replacementSlot(const ManPt* p, const ManPt& cand)
{
    int deepest = -1;
    float deepestPen = -cand.dist;
#pragma unroll
    for (int i = 0; i < kMaxManifold; i++) {
        const float pen = -p[i].dist;
        if (pen > deepestPen) { deepest = i; deepestPen = pen; }
    }
    float area[4] = { 0.f, 0.f, 0.f, 0.f };
    if (deepest != 0) area[0] = lensq(cross(cand.carPos - p[1].carPos, p[3].carPos - p[2].carPos));
    if (deepest != 1) area[1] = lensq(cross(cand.carPos - p[0].carPos, p[3].carPos - p[2].carPos));
    if (deepest != 2) area[2] = lensq(cross(cand.carPos - p[0].carPos, p[3].carPos - p[1].carPos));
    if (deepest != 3) area[3] = lensq(cross(cand.carPos - p[0].carPos, p[2].carPos - p[1].carPos));
    int best = 0;
#pragma unroll
    for (int i = 1; i < 4; i++)
        if (area[i] > area[best]) best = i;
    return best;
}

DI void addManifold(ManPt* pts, int& n, const ManPt& p)
{
    const int idx = n == kMaxManifold ? replacementSlot(pts, p) : n;
    if (n < kMaxManifold) n++;
#pragma unroll
    for (int i = 0; i < kMaxManifold; i++) pts[i] = sel(i == idx, p, pts[i]);
}

DI bool clampEdgeNormal(V3 edgeAxis, V3 faceN, V3 contactN, float edgeAngle, V3& out)
{
    V3 ec = cross(edgeAxis, faceN);
    const float cl = lensq(ec);
    if (cl <= 1e-12f) return false;
    ec = ec * rsqrt_(cl);
    const float cur = atan2_(dot(contactN, ec), dot(contactN, faceN));
    const bool outside = edgeAngle < 0.f ? cur < edgeAngle : cur > edgeAngle;
    if (!outside) return false;
    out = rodrigues(contactN, edgeAxis, edgeAngle - cur);
    return true;
}

// internal-edge normal correction of the selected arena contact (Clip.cuh:91-161)
DI void adjustEdgeContact(const LocalTri& t, V3 angles, Contact& ct)
{
    if (angles.x >= kBoundaryEdge && angles.y >= kBoundaryEdge && angles.z >= kBoundaryEdge) return;
    const V3 faceN = normalize(cross(t.e0, t.v2 - t.v0));
    int bestEdge = -1;
    float bestSq = kFltMax;
#pragma unroll
    for (int e = 0; e < 3; e++) {
        if (fabsf(comp(angles, e)) >= kBoundaryEdge) continue;
        const V3 s = triVert(t, e), en = triVert(t, e == 2 ? 0 : e + 1);
        const V3 seg = en - s;
        const float proj = dot(ct.arenaPos - s, seg) / lensq(seg);
        const V3 nearest = s + seg * clamp_(proj, 0.f, 1.f);
        const float sq = lensq(ct.arenaPos - nearest);
        if (sq < bestSq) { bestSq = sq; bestEdge = e; }
    }
    if (bestEdge < 0 || bestSq >= 5.f * 5.f) return;
    const V3 localN = normalize(ct.normal);
    const float angle = comp(angles, bestEdge);
    if (angle == 0.f) {
        if (dot(faceN, localN) >= 0.f) {
            ct.normal = faceN;
            ct.arenaPos = ct.carPos + faceN * ct.depth;
        }
        return;
    }
    const float side = angle > 0.f ? 1.f : -1.f;
    const V3 edgeAxis = normalize(triEdge(t, bestEdge));
    const V3 nA = faceN * side;
    const V3 nB = rodrigues(faceN, edgeAxis, angle) * side;
    if (dot(localN, nA) < 0.f && dot(localN, nB) < 0.f) {
        if (dot(faceN, localN) >= 0.f) {
            ct.normal = faceN;
            ct.arenaPos = ct.carPos + faceN * ct.depth;
        }
        return;
    }
    V3 cl;
    if (clampEdgeNormal(edgeAxis, nA, localN, angle, cl) && dot(cl, faceN) > 0.f) {
        ct.normal = normalize(cl);
        ct.arenaPos = ct.carPos + ct.normal * ct.depth;
    }
}

DI bool nearPoints(const V3* pos, int n, V3 carPos)
{
    bool near = false;
#pragma unroll
    for (int i = 0; i < kMaxManifold; i++)
        if (i < n && lensq(pos[i] - carPos) < kManifoldBreakSq) near = true;
    return near;
}

// Contacts of one overlapping triangle in generation order (edge contact, or
// the clipped triangle's vertices against the SAT face); keeps the first with
// the smallest -depth among those not within break distance of the plane
// points `near`.  bestVal starts at kFltMax; returns whether one was kept.
DI bool triBestContact(const LocalTri& t, const Sat& s, const V3* near, int nNear, Contact& best, float& bestVal)
{
    bool found = false;
    if (s.axisIdx >= 4) {
        const Contact c = edgeContact(t, s.minPen, s.axisIdx, s.minAxis);
        if (!nearPoints(near, nNear, c.carPos) && -c.depth < bestVal) {
            bestVal = -c.depth;
            best = c;
            found = true;
        }
        return found;
    }
    Poly poly;
    poly.v[0] = t.v0; poly.v[1] = t.v1; poly.v[2] = t.v2;
#pragma unroll
    for (int j = 3; j < kMaxPolygon; j++) poly.v[j] = kZero;
    poly.n = 3;
    const int faceAxis = argmax3(vabs(s.minAxis));
    // a loop, not unrolled: six inlined copies of the clip cost the kernel
    // code size for no speed
#pragma unroll 1
    for (int a = 0; a < 3; a++) {
        if (a == faceAxis) continue;
#pragma unroll
        for (int sg = 1; sg >= -1; sg -= 2) {
            if (poly.n > 0) poly = clipPolygon(poly, unitAxis(a) * (float)sg, comp(kHalf, a));
        }
    }
    const V3 faceNormal = unitAxis(faceAxis) * -copysignf(1.f, comp(s.minAxis, faceAxis));
    const float faceDist = comp(kHalf, faceAxis);
    const float minDepth = -(s.minPen + kContactBreak);
#pragma unroll
    for (int k = 0; k < kMaxPolygon; k++) {
        if (k >= poly.n) break;
        float depth = dot(faceNormal, poly.v[k]) - faceDist;
        depth = fmax_(depth, minDepth);
        if (depth > kContactBreak) continue;
        const Contact c{ poly.v[k] + s.minAxis * depth, poly.v[k], s.minAxis, -depth };
        if (!nearPoints(near, nNear, c.carPos) && -c.depth < bestVal) {
            bestVal = -c.depth;
            best = c;
            found = true;
        }
    }
    return found;
}

// Analytic arena planes (floor, ceiling, side walls) into the manifold.
DI int planeManifold(V3 cen, Q4 rot, ManPt* pts)
{
    int n = 0;
#pragma unroll
    for (int p = 0; p < 4; p++) {
        const V3 nrm = p == 0 ? kZ : (p == 1 ? V3{ 0.f, 0.f, -1.f } : (p == 2 ? kX : V3{ -1.f, 0.f, 0.f }));
        const float off = p == 0 ? 0.f : (p == 1 ? -2044.f : -4096.f);
        // the box's deepest corner lies within |kHalf| (76.6 uu, taken as 80)
        // of its centre: a centre farther from the plane than that plus the
        // contact break gives no point (a wave with no car near a plane skips it)
        if (dot(nrm, cen) - off >= 80.f + kContactBreak) continue;
        const V3 dir = unrotate(rot, -nrm);
        const V3 carPos{ dir.x >= 0 ? kHalf.x : -kHalf.x, dir.y >= 0 ? kHalf.y : -kHalf.y, dir.z >= 0 ? kHalf.z : -kHalf.z };
        const V3 worldCar = cen + rotate(rot, carPos);
        const float dist = dot(nrm, worldCar) - off;
        if (dist < kContactBreak && !nearManifold(pts, n, carPos))
            addManifold(pts, n, ManPt{ carPos, worldCar - nrm * dist, nrm, dist });
    }
    return n;
}

// Order key of a contact value (-depth) for the cooperative search: float
// order, with -0 taken as +0 (the sequential comparison treats them equal),
// then the candidate position, so the minimum is the first in cell order.
DI unsigned long long contactKey(float value, int item)
{
    if (value == 0.f) value = 0.f;
    const uint32_t u = __float_as_uint(value);
    const uint32_t ord = (u & 0x80000000u) ? ~u : (u | 0x80000000u);
    return ((unsigned long long)ord << 32) | (uint32_t)item;
}

// Manifold = arena planes plus the deepest triangle contact (Manifold.cuh:198-310).
// bestRef is the cell reference holding the deepest contact (found by the
// cooperative search of the contact kernel), -1 for none; its contact is
// regenerated here exactly as the search produced it.
// The car-arena manifold: the analytic plane points, then the deepest
// triangle contact found by the contact search (Manifold.cuh; the search
// hands over the point exactly as it would be regenerated from its triangle).
DI int buildManifold(V3 cen, Q4 rot, bool hasBest, const ManPt& best, ManPt* pts)
{
    int n = planeManifold(cen, rot, pts);
    if (hasBest) addManifold(pts, n, best);
    return n;
}

// ------------------------------------------------ cooperative cell search
//
// One wave searches the cell runs of its cars together, in two stages that
// each keep all 64 lanes busy:
//   screen every (car, cell triangle) item against bounds that prove the
//          float tests of the next stage reject it; the others are queued in
//          run order;
//   heavy  queued items, 64 at a time: the four suspension rays and the
//          box-triangle SAT; SAT hits are ranked in run order and the first
//          kMaxTriHits of each car generate their contacts.
// Per wheel the nearest ray hit is kept by an LDS atomic minimum of
// (distance, position in the run): the sequential walk keeps strictly nearer
// hits, so this is its result.  Contacts compete by contactKey, whose minimum
// is the first deepest contact of the walk.
//
// Screening is exact, not approximate: an item is dropped only when bounds
// from the rounding analysis of the heavy stage's float tests (arena.cpp)
// prove that both reject it:
//   SAT    the car takes no part in the car-arena search, or the triangle's
//          box, projected on one of the car's box axes, lies more than
//          kSatMargin beyond the box face (the float SAT tests those axes on
//          rotated vertices whose rounding stays below 0.25 within the
//          screening range), or the car box lies beyond the triangle's plane
//          by more than the deviation bound of the float normal axis allows;
//   rays   the segments of all four rays keep a distance beyond the
//          triangle's plane tolerance from its plane, or the triangle's box
//          lies a gap G beyond their box with |n.dir| (G - kGapSlack) above
//          its conditioning bound: an accepted hit lies within those bounds
//          of the plane and of the triangle.
// Cars outside the screening range (|position| >= kScreenRange on an axis, or
// a degenerate quaternion) are not screened.
constexpr float kSatMargin = 0.5f;
constexpr float kGapSlack = 0.05f;
constexpr float kPlaneSlack = 0.05f;
constexpr float kScreenRange = 8192.f;
constexpr float kRotErr = 100.f * 0x1p-24f;    // rotated vertex error per unit of distance (96 eps, rounded up)
constexpr float kRotErr2 = 2.f * kRotErr;      // the same for an edge (two vertices)
constexpr float kHalfLen = 80.f;               // |kHalf| rounded up

// Cars searched per wave (owner lanes 0..Owners-1); the other lanes only
// take part in the cooperative item loop.  The per-owner LDS is sized for the
// owners alone.  The contact kernel searches kContactOwners cars per wave,
// which keeps its block's LDS small enough that its occupancy is set by its
// registers; the tick-window kernel searches a whole wave of cars at once.
constexpr int kContactOwners = 32;

constexpr int kQueueSat = 1 << 23;   // queue entry flag; item positions stay below it (kMaxArenaTris)

template <int Owners>
struct ContactLdsT {
    int excl[64];
    int first[Owners];   // first reference of the owner's run
    int fine[Owners];    // the run is a candidate-grid list (else a broadphase cell's)
    int bcell[Owners];   // the owner's broadphase cell, x | y << 6 | z << 12
    int satOn[Owners];   // owner takes part in the car-arena search (not demoed)
    float rot[4][Owners];
    // screening, per owner: (cen, rayLo.x) (ax, rayLo.y) (ay, rayLo.z)
    // (az, rayHi.x) (rayHi.y, rayHi.z, screened, satOn); ax..az are the car's
    // box axes, ray* the box of the four ray segments
    float4 scr[5][Owners];
    float nearPos[kMaxManifold][3][Owners];
    int nearN[Owners];
    int satHits[Owners];
    unsigned long long rayKey[kWheels][Owners];
    unsigned long long bestKey[Owners];
    float rayNrm[kWheels][3][Owners];   // surface normal of each wheel's nearest arena hit
    float bestPt[10][Owners];           // manifold point of the deepest arena contact so far
    // screened items in run order, entries owner << 24 | kQueueSat (the SAT
    // may accept it) | triangle
    int candQ[128];
    int candN;
};
using ContactLds = ContactLdsT<kContactOwners>;

constexpr unsigned long long kNoKey = ~0ull;

template <int Owners>
DI V3 ownerCen(const ContactLdsT<Owners>& L, int o)
{
    const float4 c = L.scr[0][o];
    return V3{ c.x, c.y, c.z };
}
// suspension ray direction: minus the car's up axis
template <int Owners>
DI V3 ownerDir(const ContactLdsT<Owners>& L, int o)
{
    const float4 a = L.scr[3][o];
    return V3{ -a.x, -a.y, -a.z };
}

struct RefBox {
    float4 lo, hi, pl, sat;
    bool live;   // an item of the owner's broadphase cell
    int tri;     // the triangle
};

// Whether a triangle with packed registration range `reg` (x0 x1 y0 y1 6 bits
// each, z0 z1 4 bits) is listed in the broadphase cell `bcell`.
DI bool registeredIn(uint32_t reg, int bcell)
{
    const int x = bcell & 63, y = (bcell >> 6) & 63, z = bcell >> 12;
    return (int)(reg & 63) <= x && x <= (int)((reg >> 6) & 63) && (int)((reg >> 12) & 63) <= y &&
           y <= (int)((reg >> 18) & 63) && (int)((reg >> 24) & 15) <= z && z <= (int)(reg >> 28);
}

// The triangle of item q of owner o's run: an entry of a car-grid list or of
// a broadphase cell's run (both in ascending triangle order).
template <int Owners>
DI int contactIndex(const Dev& d, const ContactLdsT<Owners>& L, int o, int q, bool valid)
{
    const int ref = valid ? L.first[o] + q : 0;
    return (L.fine[o] ? d.arena.carTri : d.arena.cellTri)[ref];
}

// The screening data of triangle `tri` for owner o, from the per-triangle
// tables (triangle 0 for lanes without an item).  An item of a candidate-grid
// run counts only when the triangle is listed in the owner's broadphase cell:
// the reference tests exactly the triangles of that cell.
template <int Owners>
DI RefBox contactFetchTri(const Dev& d, const ContactLdsT<Owners>& L, int tri, int o, bool valid)
{
    const int t = valid ? tri : 0;
    const float4* b = d.arena.triBox + 4 * (size_t)t;
    bool live = valid;
    if (L.fine[o]) live = live && registeredIn(__float_as_uint(d.arena.triAux[t].w), L.bcell[o]);
    return RefBox{ b[0], b[1], b[2], b[3], live, t };
}

// Both in one dependent fetch (paths off the tick's critical path).
template <int Owners>
DI RefBox contactFetch(const Dev& d, const ContactLdsT<Owners>& L, int o, int q, bool valid)
{
    return contactFetchTri(d, L, contactIndex(d, L, o, q, valid), o, valid);
}

DI void waveSync()
{
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

DI unsigned long long lanesBelow(int lane) { return lane ? (~0ull >> (64 - lane)) : 0ull; }

DI bool boxAxisMiss(V3 axis, V3 w, V3 half, float face)
{
    return fabsf(dot(axis, w)) - dot(vabs(axis), half) > face + kSatMargin;
}

// screen stage: queue the item unless the heavy stage provably rejects it
template <int Owners>
DI void contactScreen(ContactLdsT<Owners>& L, const RefBox& b, int o, int lane)
{
    const float4 s0 = L.scr[0][o], s1 = L.scr[1][o], s2 = L.scr[2][o], s3 = L.scr[3][o], s4 = L.scr[4][o];
    const V3 tlo{ b.lo.x, b.lo.y, b.lo.z }, thi{ b.hi.x, b.hi.y, b.hi.z };
    const V3 rlo{ s0.w, s1.w, s2.w }, rhi{ s3.w, s4.x, s4.y };
    const V3 az{ s3.x, s3.y, s3.z };
    const V3 w = (tlo + thi) * 0.5f - V3{ s0.x, s0.y, s0.z };
    const V3 half = (thi - tlo) * 0.5f;
    const V3 ax{ s1.x, s1.y, s1.z }, ay{ s2.x, s2.y, s2.z };
    const V3 n{ b.lo.w, b.hi.w, b.pl.x };
    // the car box against the triangle's plane, within the normal axis bound
    const float dist = l1norm(w) + l1norm(half);
    const float dev = kRotErr2 * dist + b.sat.w;
    const float dn = (dev * b.sat.x + dev * dev * b.sat.y) + b.sat.z;
    const float boxR = dot(vabs(V3{ dot(n, ax), dot(n, ay), dot(n, az) }), kHalf);
    const float planeGap = fabsf(b.pl.y - dot(n, V3{ s0.x, s0.y, s0.z })) - boxR;
    const float planeTol = (dn * (dist + kHalfLen) + kRotErr * dist) + kPlaneSlack;
    const bool satMiss = s4.w == 0.f || boxAxisMiss(ax, w, half, kHalf.x) || boxAxisMiss(ay, w, half, kHalf.y) ||
                         boxAxisMiss(az, w, half, kHalf.z) || (dn <= 0.5f && planeGap > planeTol);
    const float gap = fmax_(fmax_(fmax_(tlo.x - rhi.x, rlo.x - thi.x), fmax_(tlo.y - rhi.y, rlo.y - thi.y)),
                            fmax_(tlo.z - rhi.z, rlo.z - thi.z));
    const float cosDir = fabsf(dot(n, az)) - 1e-6f;
    const float sc = dot(n, (rlo + rhi) * 0.5f) - b.pl.y;
    const float sh = dot(vabs(n), (rhi - rlo) * 0.5f);
    const bool rayMiss = (gap > kGapSlack && cosDir * (gap - kGapSlack) > b.pl.z) || sc - sh > b.pl.w ||
                         sc + sh < -b.pl.w;
    const bool keep = b.live && (s4.z == 0.f || !(satMiss && rayMiss));
    const unsigned long long m = __ballot(keep);
    const int n0 = L.candN;
    // bit 23: the SAT may accept the item (the screen could not prove it
    // rejects; only the rays keep the others)
    const int satBit = (s4.z == 0.f || !satMiss) ? kQueueSat : 0;
    if (keep) L.candQ[n0 + __popcll(m & lanesBelow(lane))] = (o << 24) | satBit | b.tri;
    if (lane == (int)__builtin_ctzll(__ballot(1))) L.candN = n0 + __popcll(m);
}

// heavy stage for the first min(candN, 64) queued items; the rest move up.
// Queue entries are in run order, so one owner's entries in a chunk sit on
// consecutive lanes.  SAT hits within the owner's first kMaxTriHits generate
// their contacts here; each wheel's nearest ray hit so far leaves its normal
// in LDS, so the owner needs no triangle load afterwards.  An owner's run is
// in ascending triangle order, so its triangle indices order its items as
// their run positions do: the minima keyed by triangle break ties as a
// sequential walk of the run keeps its first hit.
template <int Owners>
DI void contactHeavy(const Dev& d, ContactLdsT<Owners>& L, int lane)
{
    const int n = L.candN;
    const int take = n < 64 ? n : 64;
    const bool active = lane < take;
    const int e = active ? L.candQ[lane] : 0;
    const int o = e >> 24, q = e & (kQueueSat - 1);   // q: the triangle
    const bool satNeeded = (e & kQueueSat) != 0;
    bool rayHit = false;
    V3 fn = kZero;   // surface normal facing against the rays, for lanes with a ray hit
    bool hasContact = false;
    ManPt manPt{};   // this lane's contact as a manifold point
    if (active) {
        const Tri t = loadTriIdx(d.arena, q);
        // the edge angles a contact's edge adjustment needs, loaded with the
        // triangle (one round trip instead of two)
        const float4 ang = d.arena.triAux[q];
        const V3 dir = ownerDir(L, o);
        const V3 pv = cross(dir, t.e2);
        const float det = dot(t.e1, pv);
        if (!(fabsf(det) < 1e-8f)) {
            const float invDet = 1.f / det;
            // the owner's ray starts, computed as contactPrepare computed them
            const Q4 orot{ L.rot[0][o], L.rot[1][o], L.rot[2][o], L.rot[3][o] };
            const V3 ocen = ownerCen(L, o);
#pragma unroll
            for (int k = 0; k < kWheels; k++) {
                const V3 st = wheelStart(ocen, orot, k);
                const V3 tv = st - t.v0;
                const float u = invDet * dot(tv, pv);
                if (u < 0.f || u > 1.f) continue;
                const V3 qv = cross(tv, t.e1);
                const float v = invDet * dot(dir, qv);
                if (v < 0.f || u + v > 1.f) continue;
                const float hd = invDet * dot(t.e2, qv);
                if (hd <= 0.f || hd >= wheelRay(k) + 1.f) continue;
                rayHit = true;
                atomicMin(&L.rayKey[k][o], ((unsigned long long)__float_as_uint(hd) << 32) | (uint32_t)q);
            }
        }
        // arena triangles are non-degenerate (|e1 x e2|^2 > 1e-12 is checked
        // when the mesh is built), so the first branch is the one taken
        if (rayHit) {
            fn = cross(t.e1, t.e2);
            const float nl = lensq(fn);
            if (nl > 1e-12f) {
                fn = fn * rsqrt_(nl);
                if (dot(fn, dir) > 0.f) fn = -fn;
            } else {
                fn = -dir;
            }
        }
        bool hit = false;
        LocalTri lt;
        Sat sat;
        if (L.satOn[o] && !t.plane && satNeeded) {
            const Q4 rot{ L.rot[0][o], L.rot[1][o], L.rot[2][o], L.rot[3][o] };
            lt = toLocal(t, ownerCen(L, o), rot);
            sat = boxTriSat(lt);
            hit = sat.overlap;
        }
        // rank among the owner's hits so far: earlier chunks + lower lanes of
        // the owner's lane segment in this chunk
        const int prevOwner = lane > 0 ? L.candQ[lane - 1] >> 24 : -1;
        const unsigned long long starts = __ballot(o != prevOwner);
        const unsigned long long upto = lane == 63 ? ~0ull : ((2ull << lane) - 1);
        const int segStart = 63 - __clzll(starts & upto);
        const unsigned long long hits = __ballot(hit);
        const int rank = L.satHits[o] + __popcll(hits & lanesBelow(lane) & (~0ull << segStart));
        if (hit) atomicAdd(&L.satHits[o], 1);
        if (hit && rank < kMaxTriHits) {
            V3 near[kMaxManifold];
#pragma unroll
            for (int i = 0; i < kMaxManifold; i++)
                near[i] = V3{ L.nearPos[i][0][o], L.nearPos[i][1][o], L.nearPos[i][2][o] };
            Contact c;
            float value = kFltMax;
            if (triBestContact(lt, sat, near, L.nearN[o], c, value)) {
                atomicMin(&L.bestKey[o], contactKey(value, q));
                const Q4 rot{ L.rot[0][o], L.rot[1][o], L.rot[2][o], L.rot[3][o] };
                adjustEdgeContact(lt, V3{ ang.x, ang.y, ang.z }, c);
                manPt = ManPt{ c.carPos, ownerCen(L, o) + rotate(rot, c.arenaPos), rotate(rot, c.normal), -c.depth };
                hasContact = true;
            }
        }
    }
    waveSync();
    // the lane holding a wheel's current winner (its item is the key's low
    // word, unique within the owner's run) records the winner's normal
    if (rayHit) {
#pragma unroll
        for (int k = 0; k < kWheels; k++) {
            if ((uint32_t)L.rayKey[k][o] != (uint32_t)q) continue;
            L.rayNrm[k][0][o] = fn.x; L.rayNrm[k][1][o] = fn.y; L.rayNrm[k][2][o] = fn.z;
        }
    }
    // likewise the lane holding the deepest contact so far
    if (hasContact && (uint32_t)L.bestKey[o] == (uint32_t)q) {
        const float v[10] = { manPt.carPos.x,      manPt.carPos.y,      manPt.carPos.z,      manPt.worldPos.x,
                              manPt.worldPos.y,    manPt.worldPos.z,    manPt.worldNormal.x, manPt.worldNormal.y,
                              manPt.worldNormal.z, manPt.dist };
#pragma unroll
        for (int i = 0; i < 10; i++) L.bestPt[i][o] = v[i];
    }
    const int rest = n - take;
    const int moved = lane < rest ? L.candQ[take + lane] : 0;
    waveSync();
    if (lane < rest) L.candQ[lane] = moved;
    if (lane == 0) L.candN = rest;
    waveSync();
}

// after each screen round: drain full chunks; after the last, drain everything
template <int Owners>
DI void contactDrain(const Dev& d, ContactLdsT<Owners>& L, int lane, bool last)
{
    waveSync();
    while (L.candN >= 64 || (last && L.candN > 0)) contactHeavy(d, L, lane);
}

// Owner side, before the search: pose, rays and (with sat) the plane points
// of the car-arena search into LDS.  Lanes past the owners only reset the queue.
template <int Owners>
DI void contactPrepare(ContactLdsT<Owners>& L, int lane, bool sat, V3 cen, Q4 rot, int first, bool fine, int bcell,
                       bool screen)
{
    if (lane == 0) L.candN = 0;
    if (lane >= Owners) return;
    const V3 dir = -rotate(rot, kZ);
    L.first[lane] = first;
    L.fine[lane] = fine;
    L.bcell[lane] = bcell;
    L.satOn[lane] = sat;
    L.rot[0][lane] = rot.x; L.rot[1][lane] = rot.y; L.rot[2][lane] = rot.z; L.rot[3][lane] = rot.w;
    const V3 ax = rotate(rot, kX), ay = rotate(rot, kY), az = rotate(rot, kZ);
    V3 lo{ kFltMax, kFltMax, kFltMax }, hi{ -kFltMax, -kFltMax, -kFltMax };
#pragma unroll
    for (int k = 0; k < kWheels; k++) {
        const V3 st = wheelStart(cen, rot, k);
        const V3 en = st + dir * (wheelRay(k) + 1.f);
        lo = vmin(lo, vmin(st, en));
        hi = vmax(hi, vmax(st, en));
        L.rayKey[k][lane] = kNoKey;
    }
    const bool screened = screen && fabsf(cen.x) < kScreenRange && fabsf(cen.y) < kScreenRange &&
                          fabsf(cen.z) < kScreenRange && qdot(rot, rot) > 0.25f;
    L.scr[0][lane] = make_float4(cen.x, cen.y, cen.z, lo.x);
    L.scr[1][lane] = make_float4(ax.x, ax.y, ax.z, lo.y);
    L.scr[2][lane] = make_float4(ay.x, ay.y, ay.z, lo.z);
    L.scr[3][lane] = make_float4(az.x, az.y, az.z, hi.x);
    L.scr[4][lane] = make_float4(hi.y, hi.z, screened ? 1.f : 0.f, sat ? 1.f : 0.f);
    ManPt pts[kMaxManifold];
#pragma unroll
    for (int i = 0; i < kMaxManifold; i++) pts[i] = ManPt{ kZero, kZero, kZero, 0.f };
    L.nearN[lane] = sat ? planeManifold(cen, rot, pts) : 0;
#pragma unroll
    for (int i = 0; i < kMaxManifold; i++) {
        L.nearPos[i][0][lane] = pts[i].carPos.x; L.nearPos[i][1][lane] = pts[i].carPos.y;
        L.nearPos[i][2][lane] = pts[i].carPos.z;
    }
    L.satHits[lane] = 0;
    L.bestKey[lane] = kNoKey;
}

// Owner side, after the search: wheel hits (arena winner, then cars and the
// ball: bodies(start, dir, w) casts the rays at those) and the
// triangle of the deepest arena contact (-1 for none).
template <int Owners, class Bodies>
DI int contactFinishWith(const ContactLdsT<Owners>& L, int lane, V3 cen, Q4 rot, Wheels& w, Bodies bodies)
{
    const V3 up = rotate(rot, kZ);
    const V3 dir = -up;
    V3 start[kWheels];
#pragma unroll
    for (int k = 0; k < kWheels; k++) {
        w.dist[k] = wheelRay(k) + 1.f;
        w.normal[k] = up;
        w.src[k] = kSrcNone;
        start[k] = wheelStart(cen, rot, k);
        const unsigned long long key = L.rayKey[k][lane];
        if (key == kNoKey) continue;
        w.dist[k] = __uint_as_float((uint32_t)(key >> 32));
        w.src[k] = kSrcArena;
        w.normal[k] = V3{ L.rayNrm[k][0][lane], L.rayNrm[k][1][lane], L.rayNrm[k][2][lane] };
    }
    bodies(start, dir, w);
    const unsigned long long best = L.bestKey[lane];
    return best == kNoKey ? -1 : (int)(uint32_t)best;
}

template <int Owners>
DI int contactFinish(const Dev& d, const ContactLdsT<Owners>& L, int lane, int car, int sim, V3 cen, Q4 rot, Wheels& w)
{
    return contactFinishWith(L, lane, cen, rot, w,
                             [&](const V3* start, V3 dir, Wheels& ww) { raycastBodies(d, car, sim, cen, start, dir, ww); });
}

// --------------------------------------------------------------- solver body

struct Body {
    V3 pos, vel, ang, cen;
    Q4 rot;
    V3 extVel, extAng, dVel, dAng, pushVel, turnVel;
};

DI Body makeBody(V3 pos, V3 vel, V3 ang, V3 cen, Q4 rot)
{
    Body b;
    b.pos = pos; b.vel = vel; b.ang = ang; b.cen = cen; b.rot = rot;
    b.extVel = kGravity * kDt;
    b.extAng = kZero; b.dVel = kZero; b.dAng = kZero; b.pushVel = kZero; b.turnVel = kZero;
    return b;
}

DI V3 invInertiaWorld(Q4 rot, V3 v) { return rotate(rot, unrotate(rot, v) * kCarInvInertia); }

DI void clampCarVelocity(V3& vel, V3& ang)
{
    const float vs = lensq(vel);
    if (vs > kCarMaxSpeed * kCarMaxSpeed) vel = vel * (kCarMaxSpeed * rsqrt_(vs));
    const float as = lensq(ang);
    if (as > kCarMaxAng * kCarMaxAng) ang = ang * (kCarMaxAng * rsqrt_(as));
}

DI V3 fallbackTangent(V3 n)
{
    if (fabsf(n.z) > kSqrtHalf) {
        const float inv = rsqrt_(n.y * n.y + n.z * n.z);
        return V3{ 0.f, -n.z * inv, n.y * inv };
    }
    const float inv = rsqrt_(n.x * n.x + n.y * n.y);
    return V3{ -n.y * inv, n.x * inv, 0.f };
}

// projected Gauss-Seidel updates (include/Physics/Collision/Solver.cuh:28-60)
DI float pgsClamp(float rhs, float jacInv, float relVel, float lower, float upper, float& applied)
{
    const float prev = applied;
    const float delta = rhs - applied * 0.f - relVel * jacInv;
    applied = clamp_(prev + delta, lower, upper);
    return applied - prev;
}

DI float pgsLower(float rhs, float jacInv, float relVel, float lower, float& applied)
{
    const float prev = applied;
    const float delta = rhs - applied * 0.f - relVel * jacInv;
    applied = fmax_(prev + delta, lower);
    return applied - prev;
}

// --------------------------------------------------------------- suspension

DI float nonStickyFriction(float z)
{
    if (z <= 0.f) return 0.1f;
    if (z >= 1.f) return 1.f;
    if (z < 0.7075f) return 0.1f + (z / 0.7075f) * 0.4f;
    return 0.5f + ((z - 0.7075f) / (1.f - 0.7075f)) * 0.5f;
}

DI void applySuspension(Body& b, CarRegs& r, const Wheels& w, int tick)
{
    const float brakeTorque = r.brakePrev * (kCarMass * (14.25f + 1.f / 3.f));
    const V3 up = rotate(b.rot, kZ);
    const V3 cenOffset = b.cen - b.pos;
    const V3 fwd = rotate(b.rot, kX);
    const V3 right = rotate(b.rot, kY);
    const V3 vel0 = b.vel, ang0 = b.ang;
    const V3 angCrossUp = cross(b.ang, up);
    const float pushDt = tick <= 1 ? kPushbackDtFirst : kDt;
    V3 normalSum = kZero;
    int count = 0;
#pragma unroll
    for (int k = 0; k < kWheels; k++) {
        const float dist = w.dist[k];
        if (dist > wheelRay(k)) continue;
        const float radius = wheelRadius(k), rest = wheelRest(k);
        const float suspLen = fmin_(fmax_(dist - radius, rest - kMaxTravel), rest + kMaxTravel);
        const V3 normal = w.normal[k];
        const V3 fullRel = (cenOffset + rotate(b.rot, wheelAnchor(k))) - up * dist;
        const V3 pointVel = vel0 + cross(ang0, fullRel);
        const float projVel = dot(normal, pointVel);
        const float den = dot(normal, up);
        const float clipped = den > 0.1f ? 1.f / den : 10.f;
        const float damping = projVel * clipped < 0.f ? kDampCompression : kDampRelaxation;
        float force = ((rest - suspLen) * kSuspStiffness - damping * projVel) * clipped * wheelScale(k);
        if (force <= 0.f) force = 0.f;
        float impulse = 0.f;
        if (force != 0.f) {
            impulse = force * kDt;
            const float thr = rest + radius - kSuspSub;
            if (dist < thr) {
                const V3 ta = cross(fullRel, normal);
                const float jac = kCarInvMass + dot(invInertiaWorld(b.rot, ta), ta);
                const float jacInv = 1.f / fmax_(jac, 1e-8f);
                const float posErr = kPushbackErp * (thr - dist) / pushDt;
                float push = (posErr + -projVel) * jacInv;
                if (push < 0.f) push = 0.f;
                impulse += push * 0.25f;
            }
        }
        const V3 dv = normal * (impulse * kCarInvMass);
        V3 directAng = invInertiaWorld(b.rot, cross(fullRel, normal)) * impulse;
        V3 directVel = kZero;

        V3 axle = right;
        if (k < 2 && fabsf(r.steerPrev) > 1e-6f) {
            float sn, cs;
            sincos_(r.steerPrev, &sn, &cs);
            axle = right * cs + cross(up, right) * sn;
        }
        V3 axleDir = axle - normal * dot(axle, normal);
        const float axleSq = lensq(axleDir);
        if (axleSq > 1e-10f) {
            axleDir = axleDir * rsqrt_(axleSq);
            const V3 latRel = fullRel - up * dot(up, fullRel);
            const V3 hardVel = pointVel + angCrossUp * dist;
            const V3 curveLong = cross(axle, normal);
            const V3 fwdDir = cross(normal, axleDir);
            float curveIn = 0.f;
            const float baseFric = fabsf(dot(hardVel, axle));
            if (baseFric > 5.f) curveIn = baseFric / (fabsf(dot(hardVel, curveLong)) + baseFric);
            const float hb = r.handbrakeVal;
            float latBase = 1.f - 0.8f * clamp_(curveIn, 0.f, 1.f);
            float lonBase = 1.f;
            if (hb > 0.f) {
                latBase *= (0.1f - 1.f) * hb + 1.f;
                lonBase *= ((0.5f + 0.4f * clamp_(curveIn, 0.f, 1.f)) - 1.f) * hb + 1.f;
            }
            const float fs = r.throttleVal != 0.f ? 1.f : nonStickyFriction(normal.z);
            const float latUsed = r.latF[k], lonUsed = r.lonF[k];
            r.latF[k] = latBase * fs;
            r.lonF[k] = lonBase * fs;
            const V3 angLat = invInertiaWorld(b.rot, cross(fullRel, axleDir));
            const float jac = kCarInvMass + dot(axleDir, cross(angLat, fullRel));
            const float latJacInv = 1.f / fmax_(jac, 1e-8f);
            const float sideImp = -0.2f * dot(axleDir, pointVel) * latJacInv;
            const float lonVel = dot(fwdDir, pointVel);
            const float rolling = r.drivePrev != 0.f ? -0.75f * r.drivePrev
                                                     : clamp_(-lonVel * 113.73963f, -brakeTorque, brakeTorque);
            V3 wheelImp = axleDir * (sideImp * latUsed) + fwdDir * (rolling * lonUsed);
            wheelImp = wheelImp * ((kCarMass / 3.f) * kDt);
            directVel = wheelImp * kCarInvMass;
            directAng = directAng + invInertiaWorld(b.rot, cross(latRel, wheelImp));
        }
        b.vel = b.vel + directVel;
        b.ang = b.ang + directAng;
        b.dVel = b.dVel + dv;
        normalSum = normalSum + normal;
        count += 1;
    }

    // aggregate sticky force and auto-roll, reading the previous tick's manifold
    const bool hasRaw = r.rawThrottle != 0.f;
    const bool hasWorld = r.manCount != 0;
    V3 upDir = kZero;
    bool autoroll = false;
    if (count > 0) {
        upDir = normalSum * rsqrt_(lensq(normalSum) + 1e-16f);
        const bool fullStick = r.throttleVal != 0.f || fabsf(dot(vel0, fwd)) > kStoppingVel;
        float sticky = 0.5f;
        if (fullStick) sticky += 1.f - fabsf(upDir.z);
        b.extVel = b.extVel + upDir * (sticky * kGravity.z * kDt);
        autoroll = hasRaw && (count < kWheels || hasWorld);
    } else if (hasWorld) {
        upDir = r.manNormal;
        autoroll = hasRaw;
    }
    if (autoroll) {
        const V3 down = -upDir;
        const V3 crossRight = cross(upDir, fwd);
        const V3 crossFwd = cross(down, crossRight);
        const float rtf = 1.f - clamp_(dot(right, crossRight), 0.f, 1.f);
        const float ftf = 1.f - clamp_(dot(fwd, crossFwd), 0.f, 1.f);
        const V3 rightDir = fwd * (dot(right, upDir) >= 0.f ? -1.f : 1.f);
        const V3 fwdDir = right * (dot(fwd, upDir) >= 0.f ? 1.f : -1.f);
        b.dVel = b.dVel + down * (kAutorollForce * kDt);
        b.dAng = b.dAng + (fwdDir * ftf + rightDir * rtf) * (kAutorollTorque * kDt);
    }
    b.extVel = b.extVel + r.jumpImp;
    r.jumpImp = kZero;
    b.extAng = b.extAng + r.angImp;
    r.angImp = kZero;
}

// -------------------------------------------------------- contact solver

struct Row {
    V3 axis, relCross, angular;
    float jacInv, rhs, rhsPen, lower, upper, applied, appliedPush;
};

DI Row axisRow(Q4 rot, V3 axis, V3 relPos)
{
    Row r;
    r.axis = axis;
    r.relCross = cross(relPos, axis);
    r.angular = invInertiaWorld(rot, r.relCross);
    const float den = kCarInvMass + dot(axis, cross(r.angular, relPos));
    r.jacInv = 1.f / fmax_(den, 1e-8f);
    r.rhs = 0.f; r.rhsPen = 0.f; r.lower = 0.f; r.upper = 1e10f; r.applied = 0.f; r.appliedPush = 0.f;
    return r;
}

DI float rowVel(const Row& r, V3 lin, V3 ang) { return dot(r.axis, lin) + dot(r.relCross, ang); }

DI void solveManifold(Body& b, const ManPt* pts, int count)
{
    Row nr[kMaxManifold], fr[kMaxManifold];
    const V3 cenOffset = b.cen - b.pos;
    const V3 totalVel = b.vel + b.extVel;
    const V3 totalAng = b.ang + b.extAng;
    constexpr float invDt = 1.f / kDt;
#pragma unroll
    for (int i = 0; i < kMaxManifold; i++) {
        if (i >= count) break;
        const ManPt p = pts[i];
        const V3 relPos = cenOffset + rotate(b.rot, p.carPos);
        Row n = axisRow(b.rot, p.worldNormal, relPos);
        const float rvNoExt = rowVel(n, b.vel, b.ang);
        const float rv = rowVel(n, totalVel, totalAng);
        const float rest = fabsf(rvNoExt) < kRestitutionThresh ? 0.f : kWorldRestitution * -rvNoExt;
        const float pen = p.dist + kLinearSlop;
        float posErr = 0.f;
        if (pen <= 0.f) posErr = -pen * kContactErp * invDt;
        const float posImp = posErr * n.jacInv;
        const float velImp = (rest - rv) * n.jacInv;
        if (pen > kSplitPenThresh) n.rhs = posImp + velImp;
        else { n.rhs = velImp; n.rhsPen = posImp; }
        n.applied = 0.f * kWarmStart;
        const V3 cv = totalVel + cross(totalAng, relPos);
        V3 tan = cv - p.worldNormal * dot(p.worldNormal, cv);
        const float tl = lensq(tan);
        tan = tl > 1e-8f ? tan * rsqrt_(tl) : fallbackTangent(p.worldNormal);
        Row t = axisRow(b.rot, tan, relPos);
        t.rhs = -rowVel(t, totalVel, b.ang) * t.jacInv;
        t.upper = 0.f;
        nr[i] = n;
        fr[i] = t;
        b.dVel = b.dVel + n.axis * (kCarInvMass * n.applied);
        b.dAng = b.dAng + n.angular * n.applied;
    }
    // each loop stops at an iteration whose impulses are all exactly zero: it
    // left every body and row bit for bit as it found them, so each later
    // iteration would repeat it (the accumulators start at +0 and are never -0)
    for (int it = 0; it < kSolverIters; it++) {
        bool moved = false;
#pragma unroll
        for (int i = 0; i < kMaxManifold; i++) {
            if (i >= count) break;
            Row& r = nr[i];
            if (r.rhsPen == 0.f) continue;
            const float imp = pgsLower(r.rhsPen, r.jacInv, rowVel(r, b.pushVel, b.turnVel), r.lower, r.appliedPush);
            moved |= imp != 0.f;
            b.pushVel = b.pushVel + r.axis * (kCarInvMass * imp);
            b.turnVel = b.turnVel + r.angular * imp;
        }
        if (!moved) break;
    }
    for (int it = 0; it < kSolverIters; it++) {
        bool moved = false;
#pragma unroll
        for (int i = 0; i < kMaxManifold; i++) {
            if (i >= count) break;
            Row& r = nr[i];
            const float imp = pgsLower(r.rhs, r.jacInv, rowVel(r, b.dVel, b.dAng), r.lower, r.applied);
            moved |= imp != 0.f;
            b.dVel = b.dVel + r.axis * (kCarInvMass * imp);
            b.dAng = b.dAng + r.angular * imp;
        }
#pragma unroll
        for (int i = 0; i < kMaxManifold; i++) {
            if (i >= count) break;
            const float maxImp = kWorldFriction * nr[i].applied;
            if (maxImp <= 0.f) continue;
            Row& r = fr[i];
            r.lower = -maxImp;
            r.upper = maxImp;
            const float imp = pgsClamp(r.rhs, r.jacInv, rowVel(r, b.dVel, b.dAng), r.lower, r.upper, r.applied);
            moved |= imp != 0.f;
            b.dVel = b.dVel + r.axis * (kCarInvMass * imp);
            b.dAng = b.dAng + r.angular * imp;
        }
        if (!moved) break;
    }
}

// suspension, manifold and contact solve of one non-demoed car (Solve.cuh:286-314)
DI void solveCarArena(CarRegs& r, const Wheels& w, bool hasBest, const ManPt& best, int tick)
{
    Body b = makeBody(r.pos, r.vel, r.ang, r.cen, r.rot);
    applySuspension(b, r, w, tick);
    ManPt pts[kMaxManifold];
#pragma unroll
    for (int i = 0; i < kMaxManifold; i++) pts[i] = ManPt{ kZero, kZero, kZero, 0.f };
    const int count = buildManifold(r.cen, r.rot, hasBest, best, pts);
    if (count > 0) {
        solveManifold(b, pts, count);
        if (!(lensq(b.pushVel) == 0.f && lensq(b.turnVel) == 0.f))
            integratePose(b.pos, b.cen, b.rot, b.pushVel, b.turnVel * kSplitTurnErp);
    }
    r.manCount = count;
    r.manNormal = count > 0 ? pts[0].worldNormal : kZero;
    r.pos = b.pos;
    r.vel = (b.vel + b.extVel) + b.dVel;
    r.ang = (b.ang + b.extAng) + b.dAng;
    r.cen = b.cen;
    r.rot = b.rot;
}

}  // namespace carl
