// sim_phase.h - per-simulation device physics of one tick.
//
// Reference semantics:
//   car-car OBB SAT, clip, 2-body solve, demos and bumps
//                  include/Physics/CarCar/{SAT,Clip,Solver,Solve,Response}.cuh
//   ball vs arena  include/Physics/BallArena/{Contact,Solver,Solve}.cuh
//   ball vs car    include/Physics/CarBall/{Contact,Solve,ExtraImpulse}.cuh
//   goal line      include/Physics/Goals.cuh:6-32
//   impulse cache, demo respawn   include/Physics/FinishTick.cuh:5-141
//   boost pads     include/Physics/BoostPads.cuh:58-106
// Pairs inside a simulation keep the reference's serial order: car pairs
// (b, a) for a < b with the later car as body A, then the ball.
#pragma once

#include "car_phase.h"

namespace carl {

// ------------------------------------------------------------------ car-car

struct Box {
    V3 cen;
    Q4 rot;
};

DI Box sel(bool c, const Box& a, const Box& b)
{
    return Box{ sel(c, a.cen, b.cen),
                Q4{ c ? a.rot.x : b.rot.x, c ? a.rot.y : b.rot.y, c ? a.rot.z : b.rot.z, c ? a.rot.w : b.rot.w } };
}

DI V3 boxAxis(const Box& b, int i) { return rotate(b.rot, unitAxis(i)); }

DI V3 boxSupport(const Box& b, V3 dir)
{
    const V3 ld = unrotate(b.rot, dir);
    const V3 l{ copysignf(kHalf.x, ld.x), copysignf(kHalf.y, ld.y), copysignf(kHalf.z, ld.z) };
    return b.cen + rotate(b.rot, l);
}

DI void boxBoxAxis(V3 axis, const Box& A, const Box& B, int idx, Sat& r)
{
    const float l = lensq(axis);
    if (l < 1e-12f) return;
    axis = axis * rsqrt_(l);
    const float rA = dot(vabs(unrotate(A.rot, axis)), kHalf);
    const float cA = dot(A.cen, axis);
    const float rB = dot(vabs(unrotate(B.rot, axis)), kHalf);
    const float cB = dot(B.cen, axis);
    const float aMin = cA - rA, aMax = cA + rA, bMin = cB - rB, bMax = cB + rB;
    if (aMax < bMin || bMax < aMin) { r.overlap = false; return; }
    const float dAB = aMax - bMin, dBA = bMax - aMin;
    const float depth = fmin_(dAB, dBA);
    if (depth * (idx >= 6 ? 1.05f : 1.f) >= r.minPen) return;
    r.minPen = depth;
    r.minAxis = dAB < dBA ? -axis : axis;
    r.axisIdx = idx;
}

// 15-axis OBB separation test, face axes in Bullet units (CarCar/SAT.cuh:46-125)
DI Sat boxBoxSat(const Box& A, const Box& B)
{
    Sat r{ true, 0, kFltMax, kZero };
    V3 aa[3], ba[3];
#pragma unroll
    for (int i = 0; i < 3; i++) { aa[i] = boxAxis(A, i); ba[i] = boxAxis(B, i); }
    const V3 delta = B.cen * .02f - A.cen * .02f;
    const V3 half = kHalf * .02f;
    float al[3][3];
#pragma unroll
    for (int i = 0; i < 3; i++)
#pragma unroll
        for (int j = 0; j < 3; j++) al[i][j] = fabsf(dot(aa[i], ba[j]));
#pragma unroll
    for (int i = 0; i < 3; i++) {
        const float dist = dot(delta, aa[i]);
        const float rad = comp(half, i) + half.x * al[i][0] + half.y * al[i][1] + half.z * al[i][2];
        const float depth = (rad - fabsf(dist)) * 50.f;
        if (depth < 0.f) { r.overlap = false; return r; }
        if (depth < r.minPen) { r.minPen = depth; r.minAxis = dist > 0 ? -aa[i] : aa[i]; r.axisIdx = i; }
    }
#pragma unroll
    for (int i = 0; i < 3; i++) {
        const float dist = dot(delta, ba[i]);
        const float rad = half.x * al[0][i] + half.y * al[1][i] + half.z * al[2][i] + comp(half, i);
        const float depth = (rad - fabsf(dist)) * 50.f;
        if (depth < 0.f) { r.overlap = false; return r; }
        if (depth < r.minPen) { r.minPen = depth; r.minAxis = dist > 0 ? -ba[i] : ba[i]; r.axisIdx = 3 + i; }
    }
#pragma unroll
    for (int i = 0; i < 3; i++)
#pragma unroll
        for (int j = 0; j < 3; j++) {
            boxBoxAxis(cross(aa[i], ba[j]), A, B, 6 + i * 3 + j, r);
            if (!r.overlap) return r;
        }
    return r;
}

struct PairContact {
    V3 posA, posB, normal;
    float depth;
};

DI PairContact sel(bool c, const PairContact& a, const PairContact& b)
{
    return PairContact{ sel(c, a.posA, b.posA), sel(c, a.posB, b.posB), sel(c, a.normal, b.normal),
                        sel(c, a.depth, b.depth) };
}

// reference face clipping or support-point contact (CarCar/Clip.cuh:25-197)
DI int boxBoxContacts(const Sat& s, const Box& A, const Box& B, PairContact* out)
{
    if (s.axisIdx >= 6) {
        const V3 pA = boxSupport(A, -s.minAxis);
        const V3 pB = boxSupport(B, s.minAxis);
        out[0] = PairContact{ unrotate(A.rot, pA - A.cen), unrotate(B.rot, pB - B.cen), s.minAxis, s.minPen };
        return 1;
    }
    const bool refIsA = s.axisIdx < 3;
    const Box ref = sel(refIsA, A, B);
    const Box inc = sel(refIsA, B, A);
    const int faxis = refIsA ? s.axisIdx : s.axisIdx - 3;
    V3 refN = boxAxis(ref, faxis);
    if (dot(refN, inc.cen - ref.cen) < 0.f) refN = -refN;

    int iaxis = 0;
    V3 inorm = kZero;
    float bestAl = -1.f;
#pragma unroll
    for (int a = 0; a < 3; a++) {
        const V3 n = boxAxis(inc, a);
        const float dd = dot(n, refN);
        const float al = fabsf(dd);
        if (al <= bestAl) continue;
        bestAl = al;
        iaxis = a;
        inorm = dd > 0.f ? -n : n;
    }
    const int au = iaxis == 2 ? 0 : iaxis + 1;
    const int av = iaxis == 0 ? 2 : iaxis - 1;
    const V3 eu = boxAxis(inc, au) * comp(kHalf, au);
    const V3 ev = boxAxis(inc, av) * comp(kHalf, av);
    const V3 center = inc.cen + inorm * comp(kHalf, iaxis);
    Poly poly;
    poly.v[0] = (center - eu) - ev;
    poly.v[1] = (center + eu) - ev;
    poly.v[2] = (center + eu) + ev;
    poly.v[3] = (center - eu) + ev;
#pragma unroll
    for (int j = 4; j < kMaxPolygon; j++) poly.v[j] = kZero;
    poly.n = 4;
#pragma unroll 1   // a loop: the clip's inlined copies would cost code size
    for (int a = 0; a < 3; a++) {
        if (a == faxis || poly.n == 0) continue;
        const V3 side = boxAxis(ref, a);
        const float ext = comp(kHalf, a);
        const float maxD = dot(ref.cen, side) + ext;
        const float minD = dot(ref.cen, -side) + ext;
        poly = clipPolygon(poly, side, maxD);
        if (poly.n == 0) continue;
        poly = clipPolygon(poly, -side, minD);
    }
    const V3 refCenter = ref.cen + refN * comp(kHalf, faxis);
    int n = 0;
#pragma unroll
    for (int i = 0; i < kMaxPolygon; i++) {
        if (i >= poly.n || n >= kMaxManifold) break;
        const float depth = dot(refCenter - poly.v[i], refN);
        if (depth < -kContactBreak) continue;
        const V3 onRef = poly.v[i] + refN * depth;
        const V3 pA = refIsA ? onRef : poly.v[i];
        const V3 pB = !refIsA ? onRef : poly.v[i];
        const PairContact pc{ unrotate(A.rot, pA - A.cen), unrotate(B.rot, pB - B.cen), s.minAxis, fmax_(depth, 0.f) };
#pragma unroll
        for (int j = 0; j < kMaxManifold; j++) out[j] = sel(j == n, pc, out[j]);
        n++;
    }
    if (n > 0) return n;
    out[0] = PairContact{ unrotate(A.rot, refCenter - A.cen), unrotate(B.rot, refCenter - B.cen), s.minAxis, s.minPen };
    return 1;
}

struct PairRow {
    V3 axis, rcA, rcB, angA, angB;
    float jacInv, rhs, rhsPen, applied, appliedPush;
};

DI PairRow pairRow(const Body& A, const Body& B, V3 axis, V3 relA, V3 relB)
{
    PairRow r;
    r.axis = axis;
    r.rcA = cross(relA, axis);
    r.rcB = cross(relB, axis);
    r.angA = invInertiaWorld(A.rot, r.rcA);
    r.angB = invInertiaWorld(B.rot, r.rcB);
    const float den = 2.f * kCarInvMass + dot(axis, cross(r.angA, relA)) + dot(axis, cross(r.angB, relB));
    r.jacInv = 1.f / fmax_(den, 1e-8f);
    r.rhs = 0.f; r.rhsPen = 0.f; r.applied = 0.f; r.appliedPush = 0.f;
    return r;
}

DI float pairVel(const PairRow& r, V3 lA, V3 aA, V3 lB, V3 aB)
{
    return dot(r.axis, lA) + dot(r.rcA, aA) - dot(r.axis, lB) - dot(r.rcB, aB);
}

DI void pairPush(Body& A, Body& B, const PairRow& r, float imp, bool split)
{
    const V3 lin = r.axis * (kCarInvMass * imp);
    const V3 ga = r.angA * imp, gb = r.angB * imp;
    if (split) {
        A.pushVel = A.pushVel + lin; A.turnVel = A.turnVel + ga;
        B.pushVel = B.pushVel - lin; B.turnVel = B.turnVel - gb;
    } else {
        A.dVel = A.dVel + lin; A.dAng = A.dAng + ga;
        B.dVel = B.dVel - lin; B.dAng = B.dAng - gb;
    }
}

// 2-body sequential impulses with split penetration recovery (CarCar/Solver.cuh:187-244).
// An iteration in which every row's impulse is exactly zero leaves the
// bodies and the rows' accumulated impulses bit for bit as they were (the
// accumulators start at +0 and are never -0, so adding a zero changes no
// bit), so every later iteration would repeat it: the loops stop there, with
// the result of all kSolverIters iterations.
// The friction rows are built after the split-impulse loop: their inputs (the
// pre-solve velocities, poses and contact normals) are not changed by it, so
// the rows are the same, and they need no registers during that loop.
DI void solvePair(Body& A, Body& B, const PairContact* cts, int count)
{
    PairRow nr[kMaxManifold], fr[kMaxManifold];
#pragma unroll
    for (int i = 0; i < kMaxManifold; i++) {
        if (i >= count) break;
        const V3 relA = (A.cen - A.pos) + rotate(A.rot, cts[i].posA);
        const V3 relB = (B.cen - B.pos) + rotate(B.rot, cts[i].posB);
        PairRow n = pairRow(A, B, cts[i].normal, relA, relB);
        const float rv = pairVel(n, A.vel, A.ang, B.vel, B.ang);
        const float bounce = rv < -kRestitutionThresh ? kCarCarRestitution * -rv : 0.f;
        const float pen = fmax_(cts[i].depth - kLinearSlop, 0.f);
        n.rhs = (bounce - rv) * n.jacInv;
        n.rhsPen = pen * kContactErp / kDt * n.jacInv;
        nr[i] = n;
    }
    for (int it = 0; it < kSolverIters; it++) {
        bool moved = false;
#pragma unroll
        for (int i = 0; i < kMaxManifold; i++) {
            if (i >= count) break;
            PairRow& r = nr[i];
            const float imp = pgsLower(r.rhsPen, r.jacInv, pairVel(r, A.pushVel, A.turnVel, B.pushVel, B.turnVel), 0.f,
                                       r.appliedPush);
            moved |= imp != 0.f;
            pairPush(A, B, r, imp, true);
        }
        if (!moved) break;   // a fixed point: every later iteration would move nothing either
    }
#pragma unroll
    for (int i = 0; i < kMaxManifold; i++) {
        if (i >= count) break;
        const V3 relA = (A.cen - A.pos) + rotate(A.rot, cts[i].posA);
        const V3 relB = (B.cen - B.pos) + rotate(B.rot, cts[i].posB);
        const V3 rel = (A.vel + cross(A.ang, relA)) - (B.vel + cross(B.ang, relB));
        const float nv = dot(cts[i].normal, rel);
        V3 tan = rel - cts[i].normal * nv;
        const float tl = lensq(tan);
        const float thr = fmax_(kFltEps, nv * nv * 1e-8f);
        tan = tl > thr ? tan * rsqrt_(tl) : fallbackTangent(cts[i].normal);
        PairRow t = pairRow(A, B, tan, relA, relB);
        t.rhs = -pairVel(t, A.vel, A.ang, B.vel, B.ang) * t.jacInv;
        fr[i] = t;
    }
    for (int it = 0; it < kSolverIters; it++) {
        bool moved = false;
#pragma unroll
        for (int i = 0; i < kMaxManifold; i++) {
            if (i >= count) break;
            PairRow& r = nr[i];
            const float imp = pgsLower(r.rhs, r.jacInv, pairVel(r, A.dVel, A.dAng, B.dVel, B.dAng), 0.f, r.applied);
            moved |= imp != 0.f;
            pairPush(A, B, r, imp, false);
        }
#pragma unroll
        for (int i = 0; i < kMaxManifold; i++) {
            if (i >= count) break;
            const float maxImp = kCarCarFriction * nr[i].applied;
            if (maxImp <= 0.f) continue;
            PairRow& r = fr[i];
            const float imp = pgsClamp(r.rhs, r.jacInv, pairVel(r, A.dVel, A.dAng, B.dVel, B.dAng), -maxImp, maxImp,
                                       r.applied);
            moved |= imp != 0.f;
            pairPush(A, B, r, imp, false);
        }
        if (!moved) break;
    }
}

DI float bumpCurve(float s, float lo, float mid, float hi)
{
    if (s <= 0.f) return lo;
    if (s <= 1400.f) return lo + (mid - lo) * (s / 1400.f);
    if (s <= 2200.f) return mid + (hi - mid) * ((s - 1400.f) / 800.f);
    return hi;
}

DI bool frontHit(const PairContact* cts, int count, bool aIsBumper, V3 delta, Q4 bumperRot)
{
    if (unrotate(bumperRot, delta).x > kBumpMinForward) return true;
    bool hit = false;
#pragma unroll
    for (int i = 0; i < kMaxManifold; i++) {
        const float px = aIsBumper ? cts[i].posA.x : cts[i].posB.x;
        if (i < count && px + kHitboxOffset.x > kBumpMinForward) hit = true;
    }
    return hit;
}

DI Body loadBody(const Dev& d, int c)
{
    return makeBody(d.cv(CARL_CAR_POS, c), d.cv(CARL_CAR_VEL, c), d.cv(CARL_CAR_ANG, c), d.cv(CARL_CAR_CEN, c),
                    d.cq(CARL_CAR_ROT, c));
}

DI void storeBody(const Dev& d, int c, const Body& b)
{
    d.setv(CARL_CAR_POS, c, b.pos);
    d.setv(CARL_CAR_VEL, c, b.vel);
    d.setv(CARL_CAR_ANG, c, b.ang);
    d.setv(CARL_CAR_CEN, c, b.cen);
    d.setq(CARL_CAR_ROT, c, b.rot);
}

// one car pair; ia is body A (later car), ib body B (CarCar/Solve.cuh:63-151)
DI void carCarPair(const Dev& d, int ia, int ib, int tick)
{
    if (d.ci(CARL_CAR_DEMOED, ia) || d.ci(CARL_CAR_DEMOED, ib)) return;
    const Box A{ d.cv(CARL_CAR_CEN, ia), d.cq(CARL_CAR_ROT, ia) };
    const Box B{ d.cv(CARL_CAR_CEN, ib), d.cq(CARL_CAR_ROT, ib) };
    const float maxDist = 2.f * len(kHalf);
    if (lensq(B.cen - A.cen) > maxDist * maxDist) return;
    const Sat s = boxBoxSat(A, B);
    if (!s.overlap) return;
    PairContact cts[kMaxManifold];
    const int count = boxBoxContacts(s, A, B, cts);
    if (count == 0) return;

    // demolition check on the pre-solve state
    int demoBumper = -1, demoVictim = -1;
    const int teamA = (ia % d.nCars) < d.nBlue ? 0 : 1;
    const int teamB = (ib % d.nCars) < d.nBlue ? 0 : 1;
    if (teamA != teamB && !(s.minPen < 5.f)) {
        for (int side = 0; side < 2; side++) {
            const bool aB = side == 0;
            const int bumper = aB ? ia : ib, victim = aB ? ib : ia;
            const V3 bv = d.cv(CARL_CAR_VEL, bumper), vv = d.cv(CARL_CAR_VEL, victim);
            const V3 delta = d.cv(CARL_CAR_POS, victim) - d.cv(CARL_CAR_POS, bumper);
            const float speed = len(bv);
            if (speed < kSupersonic) continue;
            if (dot(bv, delta) <= 0.f) continue;
            const V3 velDir = bv / speed;
            const float closing = dot(bv, normalize(delta));
            if (closing <= dot(vv, velDir)) continue;
            if (!frontHit(cts, count, aB, delta, aB ? A.rot : B.rot)) continue;
            demoBumper = bumper;
            demoVictim = victim;
            break;
        }
    }

    Body bA = loadBody(d, ia), bB = loadBody(d, ib);
    const V3 preA = bA.vel, preB = bB.vel;
    solvePair(bA, bB, cts, count);
    // the bump bookkeeping words, loaded under the integration below (the
    // bump pass further down reads them; nothing in between writes them)
    const int cIdxA = d.ci(CARL_CAR_CONTACT_IDX, ia), cIdxB = d.ci(CARL_CAR_CONTACT_IDX, ib);
    const float coolA = d.cf(CARL_CAR_CONTACT_COOLDOWN, ia), coolB = d.cf(CARL_CAR_CONTACT_COOLDOWN, ib);
    const bool gndA = d.ci(CARL_CAR_ON_GROUND, ia) != 0, gndB = d.ci(CARL_CAR_ON_GROUND, ib) != 0;
    const V3 impA = d.cv(CARL_CAR_IMP, ia), impB = d.cv(CARL_CAR_IMP, ib);
    bA.vel = bA.vel + bA.dVel; bA.ang = bA.ang + bA.dAng;
    bB.vel = bB.vel + bB.dVel; bB.ang = bB.ang + bB.dAng;
    bA.pos = bA.pos + bA.pushVel * kDt;
    bB.pos = bB.pos + bB.pushVel * kDt;
    bA.rot = integrateRotation(bA.rot, bA.turnVel * kSplitTurnErp);
    bB.rot = integrateRotation(bB.rot, bB.turnVel * kSplitTurnErp);
    bA.cen = bA.pos + rotate(bA.rot, kHitboxOffset);
    bB.cen = bB.pos + rotate(bB.rot, kHitboxOffset);
    clampCarVelocity(bA.vel, bA.ang);
    clampCarVelocity(bB.vel, bB.ang);
    storeBody(d, ia, bA);
    storeBody(d, ib, bB);

    if (demoVictim >= 0) {
        V3 pos = d.cv(CARL_CAR_POS, demoVictim), cen;
        Q4 rot = d.cq(CARL_CAR_ROT, demoVictim);
        integratePose(pos, cen, rot, d.cv(CARL_CAR_VEL, demoVictim), d.cv(CARL_CAR_ANG, demoVictim));
        d.setv(CARL_CAR_POS, demoVictim, pos);
        d.setv(CARL_CAR_CEN, demoVictim, cen);
        d.setq(CARL_CAR_ROT, demoVictim, rot);
        d.seti(CARL_CAR_DEMOED, demoVictim, 1);
        d.setf(CARL_CAR_DEMO_TIMER, demoVictim, kDemoRespawnTime + kDt);
        d.seti(CARL_CAR_CONTACT_IDX, demoBumper, demoVictim);
        d.setf(CARL_CAR_CONTACT_COOLDOWN, demoBumper, kBumpCooldown);
        const uint32_t seed = (uint32_t)d.seed ^ (uint32_t)demoVictim * 0x9e3779b9u ^ (uint32_t)tick;
        d.seti(CARL_CAR_RESPAWN_IDX, demoVictim, pickIndex(seed, 4));
        d.seti(CARL_CAR_LAST_RESPAWN_DIR, demoVictim, 0);
        return;
    }

    for (int side = 0; side < 2; side++) {
        const bool aB = side == 0;
        const int bumper = aB ? ia : ib, victim = aB ? ib : ia;
        const V3 bv = aB ? preA : preB, vv = aB ? preB : preA;
        const V3 delta = (aB ? bB.pos : bA.pos) - (aB ? bA.pos : bB.pos);
        if ((aB ? cIdxA : cIdxB) == victim && (aB ? coolA : coolB) > 0.f) continue;
        if (dot(bv, delta) <= 0.f) continue;
        const float speed = len(bv);
        if (speed < 1e-6f) continue;
        const V3 velDir = bv / speed;
        const float closing = dot(bv, normalize(delta));
        if (closing <= dot(vv, velDir)) continue;
        if (!frontHit(cts, count, aB, delta, aB ? bA.rot : bB.rot)) continue;
        const bool grounded = aB ? gndB : gndA;
        const float fwdScale = grounded ? bumpCurve(closing, 5.f / 6.f, 1100.f, 1530.f)
                                        : bumpCurve(closing, 5.f / 6.f, 1390.f, 1945.f);
        const V3 up = grounded ? rotate(aB ? bB.rot : bA.rot, kZ) : kZ;
        const V3 imp = velDir * fwdScale + up * bumpCurve(closing, 2.f / 6.f, 278.f, 417.f);
        d.setv(CARL_CAR_IMP, victim, (aB ? impB : impA) + imp);
        d.seti(CARL_CAR_CONTACT_IDX, bumper, victim);
        d.setf(CARL_CAR_CONTACT_COOLDOWN, bumper, kBumpCooldown);
    }
}

// ------------------------------------------------------------- ball vs arena

struct BallContact {
    V3 point, relPos, normal;
    float depth;
    V3 reduction;
};

DI BallContact sel(bool c, const BallContact& a, const BallContact& b)
{
    return BallContact{ sel(c, a.point, b.point), sel(c, a.relPos, b.relPos), sel(c, a.normal, b.normal),
                        sel(c, a.depth, b.depth), sel(c, a.reduction, b.reduction) };
}

// closest point on a triangle (Ericson, Real-Time Collision Detection 5.1.5)
DI V3 closestOnTriangle(V3 p, V3 a, V3 b, V3 c)
{
    const V3 ab = b - a, ac = c - a;
    const V3 ap = p - a;
    const float d1 = dot(ab, ap), d2 = dot(ac, ap);
    if (d1 <= 0.f && d2 <= 0.f) return a;
    const V3 bp = p - b;
    const float d3 = dot(ab, bp), d4 = dot(ac, bp);
    if (d3 >= 0.f && d4 <= d3) return b;
    const float vc = d1 * d4 - d3 * d2;
    if (vc <= 0.f && d1 >= 0.f && d3 <= 0.f) return a + ab * (d1 / (d1 - d3));
    const V3 cp = p - c;
    const float d5 = dot(ab, cp), d6 = dot(ac, cp);
    if (d6 >= 0.f && d5 <= d6) return c;
    const float vb = d5 * d2 - d1 * d6;
    if (vb <= 0.f && d2 >= 0.f && d6 <= 0.f) return a + ac * (d2 / (d2 - d6));
    const float va = d3 * d6 - d5 * d4;
    if (va <= 0.f && d4 >= d3 && d5 >= d6) {
        const float e = d4 - d3;
        return b + (c - b) * (e / (e + d5 - d6));
    }
    const float inv = 1.f / (va + vb + vc);
    return (a + ab * (vb * inv)) + ac * (vc * inv);
}

DI bool sphereTriangle(V3 center, V3 t0, V3 t1, V3 t2, BallContact& ct)
{
    const V3 point = closestOnTriangle(center, t0, t1, t2);
    const V3 delta = center - point;
    const float dsq = lensq(delta);
    const float cr = kBallRadius + kBallArenaBreak;
    if (dsq >= cr * cr) return false;
    V3 n = cross(t1 - t0, t2 - t0);
    const float nl = lensq(n);
    if (nl < 1e-12f) return false;
    n = n * rsqrt_(nl);
    if (dsq > 1e-8f && dot(n, delta) < 0.f) n = -n;
    if (dsq > 1e-8f) n = delta * rsqrt_(dsq);
    ct.point = point;
    ct.relPos = n * -kBallRadius;
    ct.normal = n;
    ct.depth = dsq > 1e-8f ? kBallRadius - sqrtf(dsq) : kBallRadius;
    ct.reduction = ct.relPos;
    return true;
}

DI int ballReplacement(const BallContact* cs, const BallContact& cand)
{
    int deepest = -1;
    float depth = cand.depth;
#pragma unroll
    for (int i = 0; i < 4; i++)
        if (cs[i].depth > depth) { deepest = i; depth = cs[i].depth; }
    float a[4] = { 0.f, 0.f, 0.f, 0.f };
    const V3 p = cand.reduction;
    if (deepest != 0) a[0] = lensq(cross(p - cs[1].reduction, cs[3].reduction - cs[2].reduction));
    if (deepest != 1) a[1] = lensq(cross(p - cs[0].reduction, cs[3].reduction - cs[2].reduction));
    if (deepest != 2) a[2] = lensq(cross(p - cs[0].reduction, cs[3].reduction - cs[1].reduction));
    if (deepest != 3) a[3] = lensq(cross(p - cs[0].reduction, cs[2].reduction - cs[1].reduction));
    int best = 0;
#pragma unroll
    for (int i = 1; i < 4; i++)
        if (a[i] > a[best]) best = i;
    return best;
}

DI void adjustBallEdge(BallContact& ct, V3 t0, V3 t1, V3 t2, V3 angles)
{
    const V3 point = ct.point;
    int bestEdge = -1;
    float bestSq = 25.f;
#pragma unroll
    for (int e = 0; e < 3; e++) {
        if (fabsf(comp(angles, e)) >= kBoundaryEdge) continue;
        const V3 s = e == 0 ? t0 : (e == 1 ? t1 : t2);
        const V3 en = e == 0 ? t1 : (e == 1 ? t2 : t0);
        const V3 edge = en - s;
        const float t = clamp_(dot(point - s, edge) / lensq(edge), 0.f, 1.f);
        const float sq = lensq(point - (s + edge * t));
        if (sq < bestSq) { bestSq = sq; bestEdge = e; }
    }
    if (bestEdge < 0) return;
    const V3 face = normalize(cross(t1 - t0, t2 - t0));
    const float angle = comp(angles, bestEdge);
    if (angle == 0.f) {
        if (dot(face, ct.normal) >= 0.f) ct.normal = face;
        return;
    }
    const float side = angle > 0.f ? 1.f : -1.f;
    const V3 s = sel(bestEdge == 0, t0, sel(bestEdge == 1, t1, t2));
    const V3 en = sel(bestEdge == 0, t1, sel(bestEdge == 1, t2, t0));
    const V3 edgeAxis = normalize(en - s);
    const V3 nA = face * side;
    const V3 nB = rodrigues(face, edgeAxis, angle) * side;
    if (dot(ct.normal, nA) < 0.f && dot(ct.normal, nB) < 0.f) {
        if (dot(face, ct.normal) >= 0.f) ct.normal = face;
        return;
    }
    V3 cl;
    if (clampEdgeNormal(edgeAxis, nA, ct.normal, angle, cl) && dot(cl, face) > 0.f) ct.normal = normalize(cl);
}

// Add one triangle's contact to the (at most four point) reduced set.
DI void reduceBallContact(const Dev& d, V3 center, const Tri& t, BallContact* cs, int& count)
{
    BallContact ct;
    if (!sphereTriangle(center, t.v0, t.v1, t.v2, ct)) return;
    int slot;
    if (count < 4) slot = count++;
    else slot = ballReplacement(cs, ct);
    const float4 ang = d.arena.angles[t.idx];
    adjustBallEdge(ct, t.v0, t.v1, t.v2, V3{ ang.x, ang.y, ang.z });
    ct.point = (center + ct.relPos) + ct.normal * ct.depth;
#pragma unroll
    for (int i = 0; i < 4; i++) cs[i] = sel(i == slot, ct, cs[i]);
}

// Sequential gather for a ball whose distinct contact triangles do not fit
// the cooperative list (rare: only balls pressed into the goal-post mesh come
// close): triangles of the overlapped cells in ascending index
// order, taken once each (the reference merges the sorted cell lists,
// BallArena/Contact.cuh:513-594).  Each pass finds the next larger triangle
// index in contact, so no candidate array is kept.
DI int gatherBallContacts(const Dev& d, V3 center, BallContact* cs)
{
    const float ext = kBallRadius + kBallArenaBreak;
    int lo[3], hi[3];
    cellOf(center - ext, lo[0], lo[1], lo[2]);
    cellOf(center + ext, hi[0], hi[1], hi[2]);
    int count = 0, last = -1;
    for (;;) {
        int next = 0x7fffffff;
        for (int z = lo[2]; z <= hi[2]; z++)
            for (int y = lo[1]; y <= hi[1]; y++)
                for (int x = lo[0]; x <= hi[0]; x++) {
                    const int cell = flatCell(x, y, z);
                    const int e = d.arena.cellStart[cell + 1];
                    for (int r = d.arena.cellStart[cell]; r < e; r++) {
                        const Tri t = loadTri(d.arena, r);
                        if (t.idx <= last || t.idx >= next) continue;
                        BallContact ct;
                        if (sphereTriangle(center, t.v0, t.v1, t.v2, ct)) next = t.idx;
                    }
                }
        if (next == 0x7fffffff) return count;
        reduceBallContact(d, center, loadTriIdx(d.arena, next), cs, count);
        last = next;
    }
}

// ---- cooperative gather over the ball candidate grid.  A ball's candidates
// are the list of the grid cell holding its centre: every triangle whose box
// comes within reach + 1 uu of that cell, each once, in ascending triangle
// order.  The reference tests the triangles registered in the broadphase cells
// its box overlaps, merged in ascending index order, so an item counts only
// when its registration range meets the ball's cell box; then the same
// sphere test decides.  A triangle the list leaves out lies more than
// reach + 1 from the centre, where the sphere test fails: its closest point is
// a convex combination of the vertices, rounded far below 1 uu.  The lists of
// the wave's balls are walked by all 64 lanes (waveItemsPipelined); each
// round's contacts are stashed in LDS and every owner folds its own, in list
// order, into its reduced set (BallArena/Contact.cuh:513-594).
struct BallLds {
    int excl[64];
    int first[64];                  // the owner's first grid reference
    int cellLo[3][64], cellHi[3][64];  // the ball's broadphase cell box
    float cx[64], cy[64], cz[64];
    float stash[13][64];            // this round's contacts, by lane
};

// grid cell of a ball centre; false outside the grid (the sequential gather
// then serves the ball)
DI bool ballGridCell(V3 c, int& cell)
{
    const float x = (c.x - kArenaMin.x) / kFineCell;
    const float y = (c.y - kArenaMin.y) / kFineCell;
    const float z = (c.z - kArenaMin.z) / kFineCell;
    if (!(x >= 0.f && x < (float)kFineX && y >= 0.f && y < (float)kFineY && z >= 0.f && z < (float)kFineZ))
        return false;
    cell = (int)x + kFineX * ((int)y + kFineY * (int)z);
    return true;
}

DI void ballPrepare(BallLds& L, int lane, V3 center, int first)
{
    const float ext = kBallRadius + kBallArenaBreak;
    int lo[3], hi[3];
    cellOf(center - ext, lo[0], lo[1], lo[2]);
    cellOf(center + ext, hi[0], hi[1], hi[2]);
#pragma unroll
    for (int k = 0; k < 3; k++) {
        L.cellLo[k][lane] = lo[k];
        L.cellHi[k][lane] = hi[k];
    }
    L.cx[lane] = center.x;
    L.cy[lane] = center.y;
    L.cz[lane] = center.z;
    L.first[lane] = first;
}

struct BallItem {
    Tri t;
    float4 aux;   // signed edge angles xyz, packed registration range (bits)
};

// the triangle of item q of owner o (reference 0 for lanes without an item)
DI BallItem ballGatherFetch(const Dev& d, const BallLds& L, int o, int q, bool valid)
{
    const int ref = valid ? L.first[o] + q : 0;
    return BallItem{ unpackTri(d.arena.fineRec + 4 * (size_t)ref), d.arena.fineAux[ref] };
}

// Test one item; a contact is stashed at the lane's slot (true when there is one).
DI bool ballGatherItem(BallLds& L, const BallItem& item, int o, int lane)
{
    const Tri& t = item.t;
    const uint32_t r = __float_as_uint(item.aux.w);
    if ((int)(r & 63) > L.cellHi[0][o] || (int)((r >> 6) & 63) < L.cellLo[0][o] ||
        (int)((r >> 12) & 63) > L.cellHi[1][o] || (int)((r >> 18) & 63) < L.cellLo[1][o] ||
        (int)((r >> 24) & 15) > L.cellHi[2][o] || (int)(r >> 28) < L.cellLo[2][o])
        return false;
    const V3 center{ L.cx[o], L.cy[o], L.cz[o] };
    const float reach = kBallRadius + kBallArenaBreak + 1.f;
    const V3 mn = vmin(vmin(t.v0, t.v1), t.v2);
    const V3 mx = vmax(vmax(t.v0, t.v1), t.v2);
    if (center.x < mn.x - reach || center.x > mx.x + reach || center.y < mn.y - reach || center.y > mx.y + reach ||
        center.z < mn.z - reach || center.z > mx.z + reach)
        return false;
    BallContact ct;
    if (!sphereTriangle(center, t.v0, t.v1, t.v2, ct)) return false;
    adjustBallEdge(ct, t.v0, t.v1, t.v2, V3{ item.aux.x, item.aux.y, item.aux.z });
    ct.point = (center + ct.relPos) + ct.normal * ct.depth;
    const float v[13] = { ct.point.x,  ct.point.y,  ct.point.z,  ct.relPos.x,    ct.relPos.y,    ct.relPos.z,   ct.normal.x,
                          ct.normal.y, ct.normal.z, ct.depth,    ct.reduction.x, ct.reduction.y, ct.reduction.z };
#pragma unroll
    for (int i = 0; i < 13; i++) L.stash[i][lane] = v[i];
    return true;
}

// Fold the stashed contacts of lanes [a, b) marked in `hits` into the set.
DI void foldStashedContacts(const BallLds& L, unsigned long long hits, int a, int b, BallContact* cs, int& count)
{
    const unsigned long long hiMask = b >= 64 ? ~0ull : ((1ull << b) - 1);
    unsigned long long bits = hits & hiMask & (~0ull << a);
    while (bits) {
        const int i = (int)__builtin_ctzll(bits);
        bits &= bits - 1;
        BallContact ct;
        ct.point = V3{ L.stash[0][i], L.stash[1][i], L.stash[2][i] };
        ct.relPos = V3{ L.stash[3][i], L.stash[4][i], L.stash[5][i] };
        ct.normal = V3{ L.stash[6][i], L.stash[7][i], L.stash[8][i] };
        ct.depth = L.stash[9][i];
        ct.reduction = V3{ L.stash[10][i], L.stash[11][i], L.stash[12][i] };
        // the edge adjustment changes only the normal, so the replacement
        // choice sees what the reference's sees
        int slot;
        if (count < 4) slot = count++;
        else slot = ballReplacement(cs, ct);
#pragma unroll
        for (int k = 0; k < 4; k++) cs[k] = sel(k == slot, ct, cs[k]);
    }
}

struct BallBody {
    V3 vel, velNoExt, ang, dVel, dAng, pushVel, pushAng;
};

struct BRow {
    V3 axis, relCross;
    float jacInv, rhs, rhsPen, applied, appliedPush;
};

DI BRow ballRow(V3 axis, V3 relPos)
{
    BRow r;
    r.axis = axis;
    r.relCross = cross(relPos, axis);
    r.jacInv = 1.f / fmax_(kBallInvMass + kBallInvInertia * lensq(r.relCross), 1e-8f);
    r.rhs = 0.f; r.rhsPen = 0.f; r.applied = 0.f; r.appliedPush = 0.f;
    return r;
}

DI float bRowVel(const BRow& r, V3 lin, V3 ang) { return dot(r.axis, lin) + dot(r.relCross, ang); }

DI BRow ballNormalRow(const BallBody& b, V3 normal, float depth, V3 relPos, bool split)
{
    BRow r = ballRow(normal, relPos);
    const float rv = bRowVel(r, b.vel, b.ang);
    const float restv = bRowVel(r, b.velNoExt, b.ang);
    float bounce = fabsf(restv) >= kRestitutionThresh ? kBallRestitution * -restv : 0.f;
    bounce = fmax_(bounce, 0.f);
    const float posImp = fmax_(depth, 0.f) * kContactErp / kDt * r.jacInv;
    const float velImp = (bounce - rv) * r.jacInv;
    if (!split) r.rhs = velImp;
    else if (-depth > kSplitPenThresh) r.rhs = posImp + velImp;
    else { r.rhs = velImp; r.rhsPen = posImp; }
    return r;
}

DI void ballPush(BallBody& b, const BRow& r, float imp, bool split)
{
    const V3 lin = r.axis * (kBallInvMass * imp);
    const V3 ang = r.relCross * (kBallInvInertia * imp);
    if (split) { b.pushVel = b.pushVel + lin; b.pushAng = b.pushAng + ang; }
    else { b.dVel = b.dVel + lin; b.dAng = b.dAng + ang; }
}

// averaged-contact ball solve (BallArena/Solver.cuh:197-258)
DI void solveBallContacts(BallBody& b, const BallContact* cs, int count, bool wasHit)
{
    if (count == 0) return;
    BRow split[4];
    V3 totalN = kZero;
    float totalR = 0.f;
    const bool doSplit = !wasHit || count != 1 || cs[0].normal.z < 0.999f;
#pragma unroll
    for (int i = 0; i < 4; i++) {
        if (i >= count) break;
        split[i] = ballNormalRow(b, cs[i].normal, cs[i].depth, cs[i].relPos, doSplit);
        totalN = totalN + cs[i].normal;
        totalR += sqrtf(lensq(cs[i].relPos));
    }
    const float fc = (float)count;
    const V3 avgN = totalN * (1.f / fc);
    const V3 avgRel = avgN * (-totalR / fc);
    const float avgDepth = -totalR / fc;
    BRow nr = ballNormalRow(b, avgN, avgDepth, avgRel, false);
    const V3 pv = b.vel + cross(b.ang, avgRel);
    V3 tan = pv - avgN * dot(avgN, pv);
    const float tl = lensq(tan);
    tan = tl > 1e-8f ? tan * rsqrt_(tl) : fallbackTangent(avgN);
    BRow fr = ballRow(tan, avgRel);
    fr.rhs = -bRowVel(fr, b.vel, b.ang) * fr.jacInv;
    // each loop stops at an iteration whose impulses are all exactly zero (a
    // fixed point: the accumulators start at +0 and are never -0, so it left
    // every bit as it found it, and each later iteration would repeat it)
    for (int it = 0; it < kSolverIters; it++) {
        bool moved = false;
#pragma unroll
        for (int i = 0; i < 4; i++) {
            if (i >= count) break;
            BRow& r = split[i];
            if (r.rhsPen == 0.f) continue;
            const float imp = pgsLower(r.rhsPen, r.jacInv, bRowVel(r, b.pushVel, b.pushAng), 0.f, r.appliedPush);
            moved |= imp != 0.f;
            ballPush(b, r, imp, true);
        }
        if (!moved) break;
    }
    for (int it = 0; it < kSolverIters; it++) {
        const float ni = pgsLower(nr.rhs, nr.jacInv, bRowVel(nr, b.dVel, b.dAng), 0.f, nr.applied);
        bool moved = ni != 0.f;
        ballPush(b, nr, ni, false);
        const float maxImp = kBallFriction * nr.applied;
        if (maxImp > 0.f) {
            const float fi = pgsClamp(fr.rhs, fr.jacInv, bRowVel(fr, b.dVel, b.dAng), -maxImp, maxImp, fr.applied);
            moved |= fi != 0.f;
            ballPush(b, fr, fi, false);
        }
        if (!moved) break;
    }
    b.vel = b.vel + b.dVel;
    b.ang = b.ang + b.dAng;
    const float ss = lensq(b.vel);
    if (ss > kBallMaxSpeed * kBallMaxSpeed) b.vel = b.vel * (kBallMaxSpeed * rsqrt_(ss));
    const float as = lensq(b.ang);
    if (as > kBallMaxAng * kBallMaxAng) b.ang = b.ang * (kBallMaxAng * rsqrt_(as));
}

// ------------------------------------------- ball vs native arena meshes
// With CARL_ARENA_METADATA the ball meets the arena as RocketSim's native
// meshes do (BallArena/Contact.cuh:292-343, 406-470, 478-594): the native
// triangles in Bullet units, visited in native order (mesh, then position
// within the mesh), at most four contacts kept per mesh, and the four arena
// planes as analytic contacts.  Up to kNativeMaxContacts contacts per ball
// live in the environment's ball scratch, slot-major and field-major
// ((slot * kNativeSlotWords + field) * nSim + sim): first each contact's
// offset, normal and depth, then the solver's split row built from it.  One
// lane serves one ball.

constexpr int kNativeMaxContacts = 68;   // the reference's capacity: sixteen meshes of four and the planes
constexpr int kNativeSlotWords = 10;

struct NativeTri {
    V3 v0, v1, v2;
    int key, mesh, flags;
};

DI NativeTri loadNativeTri(const ArenaView& a, int idx)
{
    const float4* r = a.native + 4 * (size_t)idx;
    const float4 r0 = r[0], r1 = r[1], r2 = r[2];
    return NativeTri{ V3{ r0.x, r0.y, r0.z }, V3{ r1.x, r1.y, r1.z }, V3{ r2.x, r2.y, r2.z },
                      (int)__float_as_uint(r0.w), (int)__float_as_uint(r1.w), (int)__float_as_uint(r2.w) };
}

DI float& nativeWord(const Dev& d, int sim, int slot, int field)
{
    return d.ballScratch[(size_t)(slot * kNativeSlotWords + field) * d.nSim + sim];
}

// sphere against one native triangle, all in Bullet units
// (BallArena/Contact.cuh:292-343); reduction = relPos
DI bool nativeSphereTriangle(V3 center, const NativeTri& t, BallContact& ct)
{
    constexpr float radius = kBallRadius * .02f;
    constexpr float extent = radius + kBallArenaBreak * .02f;
    const V3 e01 = t.v1 - t.v0, e02 = t.v2 - t.v0;
    const V3 off = center - t.v0;
    const V3 face = cross(e01, e02);
    const float nl = lensq(face);
    if (nl < 1e-14f) return false;
    V3 n = face * (1.f / sqrtf(nl));
    float plane = dot(off, n);
    if (plane < 0.f) {
        plane = -plane;
        n = -n;
    }
    if (plane >= extent) return false;
    const float gamma = dot(cross(e01, off), face) / nl;
    const float beta = dot(cross(off, e02), face) / nl;
    const float alpha = 1.f - gamma - beta;
    const bool inside = alpha >= 0.f && alpha <= 1.f && beta >= 0.f && beta <= 1.f && gamma >= 0.f && gamma <= 1.f;
    const V3 point = inside ? center - n * plane : closestOnTriangle(center, t.v0, t.v1, t.v2);
    const V3 delta = center - point;
    const float dsq = lensq(delta);
    if (dsq >= extent * extent) return false;
    const float dist = sqrtf(dsq);
    ct.point = point;
    ct.normal = dsq > kFltEps ? delta * (1.f / dist) : n;
    ct.depth = dsq > kFltEps ? radius - dist : radius;
    ct.relPos = (point - ct.normal * ct.depth) - center;
    ct.reduction = ct.relPos;
    return true;
}

// native internal-edge correction (BallArena/Contact.cuh:161-202): the edge
// within 0.1 Bullet units of the contact point, its metadata flags choosing
// the sides; the clamped normal is kept as the rotation leaves it
DI void adjustNativeBallEdge(BallContact& ct, const NativeTri& t, V3 angles)
{
    const float maxSq = .1f * .1f;
    int best = -1;
    float bestSq = maxSq;
#pragma unroll
    for (int e = 0; e < 3; e++) {
        if (fabsf(comp(angles, e)) >= kBoundaryEdge) continue;
        const V3 s = e == 0 ? t.v0 : (e == 1 ? t.v1 : t.v2);
        const V3 en = e == 0 ? t.v1 : (e == 1 ? t.v2 : t.v0);
        const V3 edge = en - s;
        const float u = clamp_(dot(ct.point - s, edge) / lensq(edge), 0.f, 1.f);
        const float sq = lensq(ct.point - (s + edge * u));
        if (sq < bestSq) { bestSq = sq; best = e; }
    }
    if (best < 0) return;
    const V3 face = normalize(cross(t.v1 - t.v0, t.v2 - t.v0));
    const V3 s = sel(best == 0, t.v0, sel(best == 1, t.v1, t.v2));
    const V3 en = sel(best == 0, t.v1, sel(best == 1, t.v2, t.v0));
    const V3 edgeDir = normalize(s - en);
    const float angle = comp(angles, best);
    bool concave = angle == 0.f;
    if (!concave) {
        const float sign = (t.flags & (1 << best)) ? 1.f : -1.f;
        V3 other = rodrigues(face, edgeDir, angle);
        if (t.flags & (1 << (best + 3))) other = -other;
        concave = dot(ct.normal, face * sign) < 0.f && dot(ct.normal, other * sign) < 0.f;
        if (!concave) {
            V3 cl;
            if (clampEdgeNormal(edgeDir, face * sign, ct.normal, angle, cl) && dot(cl, face) > 0.f) ct.normal = cl;
        }
    }
    if (concave && dot(face, ct.normal) >= 0.f) ct.normal = face;
}

// a finished mesh group's contacts into their slots, back in Unreal units
DI void storeNativeGroup(const Dev& d, int sim, int base, int n, const BallContact* cs)
{
#pragma unroll
    for (int i = 0; i < 4; i++) {
        if (i >= n) break;
        const float v[7] = { cs[i].relPos.x * 50.f, cs[i].relPos.y * 50.f, cs[i].relPos.z * 50.f, cs[i].normal.x,
                             cs[i].normal.y,        cs[i].normal.z,        cs[i].depth * 50.f };
#pragma unroll
        for (int f = 0; f < 7; f++) nativeWord(d, sim, base + i, f) = v[f];
    }
}

// The native contacts of a ball centred at `center` into the ball's slots;
// returns their count.  The reference merges its cells' lists, sorted by
// order key (mesh * 10000 + order), and visits each distinct triangle once
// in that order; here each pass over the overlapped cells finds the
// smallest (key, triangle) pair above the last one visited whose triangle
// makes contact, the same sequence when keys are unique (equal keys, which
// the reference leaves in std::sort's order, go by triangle index).  The
// planes in reach are counted first; a contact that would need a slot past
// the 68 less those is dropped (the reference writes past its array there).
DI int gatherNativeBallContacts(const Dev& d, int sim, V3 center)
{
    // the arena planes: floor, ceiling, the two side walls (analytic)
    const V3 normals[4] = { V3{ 0.f, 0.f, 1.f }, V3{ 0.f, 0.f, -1.f }, V3{ 1.f, 0.f, 0.f }, V3{ -1.f, 0.f, 0.f } };
    const float offsets[4] = { 0.f, -2044.f, -4096.f, -4096.f };
    float planeDepth[4];
    int room = kNativeMaxContacts;
#pragma unroll
    for (int p = 0; p < 4; p++) {
        planeDepth[p] = kBallRadius - (dot(normals[p], center) - offsets[p]);
        room -= planeDepth[p] > -kBallArenaBreak;
    }
    const float ext = kBallRadius + kBallArenaBreak;
    int lo[3], hi[3];
    cellOf(center - ext, lo[0], lo[1], lo[2]);
    cellOf(center + ext, hi[0], hi[1], hi[2]);
    const V3 cb = center * .02f;
    BallContact cs[4];
#pragma unroll
    for (int k = 0; k < 4; k++) cs[k] = BallContact{ kZero, kZero, kZero, 0.f, kZero };
    int count = 0, local = 0, mesh = -1, base = 0;
    constexpr long long kNone = 0x7fffffffffffffffLL;
    long long last = -kNone - 1;
    for (;;) {
        long long next = kNone;
        for (int z = lo[2]; z <= hi[2]; z++)
            for (int y = lo[1]; y <= hi[1]; y++)
                for (int x = lo[0]; x <= hi[0]; x++) {
                    const int cell = flatCell(x, y, z);
                    const int e = d.arena.cellStart[cell + 1];
                    for (int r = d.arena.cellStart[cell]; r < e; r++) {
                        const int idx = (int)(__float_as_uint(d.arena.rec[4 * (size_t)r + 3].w) & ~kPlaneFlag);
                        const NativeTri t = loadNativeTri(d.arena, idx);
                        const long long k = (long long)t.key * 4294967296LL + idx;
                        if (k <= last || k >= next || t.mesh < 0) continue;
                        BallContact ct;
                        if (nativeSphereTriangle(cb, t, ct)) next = k;
                    }
                }
        if (next == kNone) break;
        last = next;
        const int idx = (int)(next & 0xffffffffLL);
        const NativeTri t = loadNativeTri(d.arena, idx);
        BallContact ct;
        nativeSphereTriangle(cb, t, ct);
        if (t.mesh != mesh) {
            storeNativeGroup(d, sim, base, local, cs);
            base = count;
            local = 0;
            mesh = t.mesh;
        }
        int slot;
        if (local < 4) {
            if (count == room) continue;
            slot = local++;
            count++;
        } else {
            slot = ballReplacement(cs, ct);
        }
        const float4 a = d.arena.native[4 * (size_t)idx + 3];
        adjustNativeBallEdge(ct, t, V3{ a.x, a.y, a.z });
#pragma unroll
        for (int i = 0; i < 4; i++) cs[i] = sel(i == slot, ct, cs[i]);
    }
    storeNativeGroup(d, sim, base, local, cs);
#pragma unroll
    for (int p = 0; p < 4; p++) {
        const float depth = planeDepth[p];
        if (!(depth > -kBallArenaBreak)) continue;
        const V3 rel = normals[p] * -kBallRadius;
        const float v[7] = { rel.x, rel.y, rel.z, normals[p].x, normals[p].y, normals[p].z, depth };
#pragma unroll
        for (int f = 0; f < 7; f++) nativeWord(d, sim, count, f) = v[f];
        count++;
    }
    return count;
}

// The averaged-contact solve of solveBallContacts over the ball's stored
// native contacts; each slot's contact is replaced by its split row (axis,
// relative cross, jacInv, rhsPen, applied push).
DI void solveNativeBallContacts(const Dev& d, int sim, BallBody& b, int count, bool wasHit)
{
    if (count == 0) return;
    V3 totalN = kZero;
    float totalR = 0.f;
    const bool doSplit = !wasHit || count != 1 || nativeWord(d, sim, 0, 5) < 0.999f;
    for (int i = 0; i < count; i++) {
        const V3 rel{ nativeWord(d, sim, i, 0), nativeWord(d, sim, i, 1), nativeWord(d, sim, i, 2) };
        const V3 n{ nativeWord(d, sim, i, 3), nativeWord(d, sim, i, 4), nativeWord(d, sim, i, 5) };
        const float depth = nativeWord(d, sim, i, 6);
        const BRow r = ballNormalRow(b, n, depth, rel, doSplit);
        totalN = totalN + n;
        totalR += sqrtf(lensq(rel));
        const float v[9] = { r.axis.x, r.axis.y, r.axis.z, r.relCross.x, r.relCross.y, r.relCross.z,
                             r.jacInv, r.rhsPen,  0.f };
#pragma unroll
        for (int f = 0; f < 9; f++) nativeWord(d, sim, i, f) = v[f];
    }
    const float fc = (float)count;
    const V3 avgN = totalN * (1.f / fc);
    const V3 avgRel = avgN * (-totalR / fc);
    const float avgDepth = -totalR / fc;
    BRow nr = ballNormalRow(b, avgN, avgDepth, avgRel, false);
    const V3 pv = b.vel + cross(b.ang, avgRel);
    V3 tan = pv - avgN * dot(avgN, pv);
    const float tl = lensq(tan);
    tan = tl > 1e-8f ? tan * rsqrt_(tl) : fallbackTangent(avgN);
    BRow fr = ballRow(tan, avgRel);
    fr.rhs = -bRowVel(fr, b.vel, b.ang) * fr.jacInv;
    // the loops stop at a fixed point, as in solveBallContacts
    for (int it = 0; it < kSolverIters; it++) {
        bool moved = false;
        for (int i = 0; i < count; i++) {
            BRow r;
            r.rhsPen = nativeWord(d, sim, i, 7);
            if (r.rhsPen == 0.f) continue;
            r.axis = V3{ nativeWord(d, sim, i, 0), nativeWord(d, sim, i, 1), nativeWord(d, sim, i, 2) };
            r.relCross = V3{ nativeWord(d, sim, i, 3), nativeWord(d, sim, i, 4), nativeWord(d, sim, i, 5) };
            r.jacInv = nativeWord(d, sim, i, 6);
            r.appliedPush = nativeWord(d, sim, i, 8);
            const float imp = pgsLower(r.rhsPen, r.jacInv, bRowVel(r, b.pushVel, b.pushAng), 0.f, r.appliedPush);
            nativeWord(d, sim, i, 8) = r.appliedPush;
            moved |= imp != 0.f;
            ballPush(b, r, imp, true);
        }
        if (!moved) break;
    }
    for (int it = 0; it < kSolverIters; it++) {
        const float ni = pgsLower(nr.rhs, nr.jacInv, bRowVel(nr, b.dVel, b.dAng), 0.f, nr.applied);
        bool moved = ni != 0.f;
        ballPush(b, nr, ni, false);
        const float maxImp = kBallFriction * nr.applied;
        if (maxImp > 0.f) {
            const float fi = pgsClamp(fr.rhs, fr.jacInv, bRowVel(fr, b.dVel, b.dAng), -maxImp, maxImp, fr.applied);
            moved |= fi != 0.f;
            ballPush(b, fr, fi, false);
        }
        if (!moved) break;
    }
    b.vel = b.vel + b.dVel;
    b.ang = b.ang + b.dAng;
    const float ss = lensq(b.vel);
    if (ss > kBallMaxSpeed * kBallMaxSpeed) b.vel = b.vel * (kBallMaxSpeed * rsqrt_(ss));
    const float as = lensq(b.ang);
    if (as > kBallMaxAng * kBallMaxAng) b.ang = b.ang * (kBallMaxAng * rsqrt_(as));
}

// --------------------------------------------------------------- ball vs car

struct BCRow {
    V3 axis, ballTorque, carAngular;
    float jacInv, applied;
};

DI BCRow bcRow(Q4 rot, V3 axis, V3 ballOff, V3 carOff)
{
    BCRow r;
    r.axis = axis;
    r.ballTorque = cross(ballOff, axis);
    const V3 ct = cross(carOff, axis);
    r.carAngular = rotate(rot, unrotate(rot, ct) * kCarInvInertia);
    const float den = kBallInvMass + kCarInvMass + kBallInvInertia * lensq(r.ballTorque) + dot(r.carAngular, ct);
    r.jacInv = 1.f / fmax_(den, 1e-8f);
    r.applied = 0.f;
    return r;
}

DI float bcVel(const BCRow& r, V3 bv, V3 ba, V3 cv, V3 ca, V3 ballOff, V3 carOff)
{
    return dot(r.axis, (bv + cross(ba, ballOff)) - (cv + cross(ca, carOff)));
}

DI float extraCurve(float s)
{
    if (s <= 500.f) return 0.65f;
    if (s <= 2300.f) return 0.65f + (0.55f - 0.65f) * ((s - 500.f) / 1800.f);
    if (s <= 4600.f) return 0.55f + (0.30f - 0.55f) * ((s - 2300.f) / 2300.f);
    return 0.30f;
}

// one ball-car contact solve, split correction and extra impulse
// (CarBall/Solve.cuh:207-243) for a car that is not demolished.  The ball's
// position and velocities are the caller's registers, updated in place (the
// caller stores them); every word of the car the pair reads, and the ball's
// accumulated impulse, is loaded in one batch before any is tested.  True
// when the pair is in contact (the ball's velocities have been solved).
DI bool ballCarPair(const Dev& d, int sim, int c, V3 preBallVel, int tick, V3& ballNow, V3& bv, V3& ba)
{
    const V3 carPos = d.cv(CARL_CAR_POS, c), carCen = d.cv(CARL_CAR_CEN, c);
    V3 cv = d.cv(CARL_CAR_VEL, c), ca = d.cv(CARL_CAR_ANG, c);
    const Q4 rot = d.cq(CARL_CAR_ROT, c);
    const int last = d.ci(CARL_CAR_BALL_HIT_TICK, c);
    const V3 ballImp = d.sv(CARL_SIM_BALL_IMP, sim);
    const V3 ballPos = ballNow;
    const V3 preCarVel = cv;

    const V3 core{ kHalf.x - kCarMargin, kHalf.y - kCarMargin, kHalf.z - kCarMargin };
    const V3 lb = unrotate(rot, ballPos - carCen);
    const V3 cl{ clamp_(lb.x, -core.x, core.x), clamp_(lb.y, -core.y, core.y), clamp_(lb.z, -core.z, core.z) };
    const V3 dl = lb - cl;
    const float dsq = lensq(dl);
    const float inter = kBallRadius + kCarMargin;
    const float accept = inter + kCarBallBreak;
    V3 point, normal;
    float depth;
    if (dsq > 1e-8f) {
        if (dsq >= accept * accept) return false;
        const float dist = sqrtf(dsq);
        const V3 ln = dl * (1.f / dist);
        point = carCen + rotate(rot, cl + ln * kCarMargin);
        normal = rotate(rot, ln);
        depth = inter - dist;
    } else {
        const V3 fd = core - vabs(lb);
        int axis = 0;
        float md = fd.x;
        if (fd.y < md) { axis = 1; md = fd.y; }
        if (fd.z < md) { axis = 2; md = fd.z; }
        V3 ln = kZero;
        setComp(ln, axis, comp(lb, axis) >= 0.f ? 1.f : -1.f);
        point = carCen + rotate(rot, cl + ln * kCarMargin);
        normal = rotate(rot, ln);
        depth = inter + md;
    }

    const V3 ballOff = normal * -kBallRadius;
    const V3 carOff = point - carPos;
    BCRow nr = bcRow(rot, normal, ballOff, carOff);
    const float relN = bcVel(nr, bv, ba, cv, ca, ballOff, carOff);
    V3 tan = (bv + cross(ba, ballOff)) - (cv + cross(ca, carOff));
    tan = tan - normal * relN;
    const float tl = lensq(tan);
    const float restitution = fabsf(relN) > kRestitutionThresh ? kCarBallRestitution * -relN : 0.f;
    tan = tl > kFltEps ? tan * rsqrt_(tl) : fallbackTangent(normal);
    BCRow fr = bcRow(rot, tan, ballOff, carOff);
    for (int it = 0; it < kSolverIters; it++) {
        const float ni = pgsLower(restitution * nr.jacInv, nr.jacInv, bcVel(nr, bv, ba, cv, ca, ballOff, carOff), 0.f,
                                  nr.applied);
        bv = bv + nr.axis * (ni * kBallInvMass);
        ba = ba + nr.ballTorque * (ni * kBallInvInertia);
        cv = cv - nr.axis * (ni * kCarInvMass);
        ca = ca - nr.carAngular * ni;
        const float maxF = kCarBallFriction * nr.applied;
        const float fi = pgsClamp(0.f, fr.jacInv, bcVel(fr, bv, ba, cv, ca, ballOff, carOff), -maxF, maxF, fr.applied);
        bv = bv + fr.axis * (fi * kBallInvMass);
        ba = ba + fr.ballTorque * (fi * kBallInvInertia);
        cv = cv - fr.axis * (fi * kCarInvMass);
        ca = ca - fr.carAngular * fi;
    }
    d.setv(CARL_CAR_VEL, c, cv);
    d.setv(CARL_CAR_ANG, c, ca);

    const float pen = depth - kLinearSlop;
    if (pen > 0.f) {
        const float push = pen * kContactErp / kDt * nr.jacInv;
        ballNow = ballPos + normal * (push * kBallInvMass * kDt);
        const V3 np = carPos + normal * (-push * kCarInvMass * kDt);
        const Q4 nrot = integrateRotation(rot, (nr.carAngular * -push) * kSplitTurnErp);
        d.setv(CARL_CAR_POS, c, np);
        d.setq(CARL_CAR_ROT, c, nrot);
        d.setv(CARL_CAR_CEN, c, np + rotate(nrot, kHitboxOffset));
    }

    d.seti(CARL_CAR_BALL_CONTACT_TICK, c, tick);
    d.sseti(CARL_SIM_LAST_TOUCH_TICK, sim, tick);
    if (tick <= last + 1 && last <= tick) return true;
    d.seti(CARL_CAR_BALL_HIT_TICK, c, tick);
    const V3 relVel = preBallVel - preCarVel;
    const float speed = fmin_(sqrtf(lensq(relVel)), kExtraMaxDv);
    V3 added = kZero;
    if (speed > 0.f) {
        const V3 rp = ballPos - carPos;
        V3 hd{ rp.x, rp.y, rp.z * kExtraZScale };
        const float hl = lensq(hd);
        if (hl > 1e-12f) {
            hd = hd * rsqrt_(hl);
            const V3 fwd = rotate(rot, kX);
            hd = hd - fwd * (dot(hd, fwd) * (1.f - kExtraFwdScale));
            const float al = lensq(hd);
            if (al > 1e-12f) hd = hd * rsqrt_(al);
            added = hd * (speed * extraCurve(speed));
        }
    }
    d.ssetv(CARL_SIM_BALL_IMP, sim, ballImp + added);
    return true;
}

// drag, arena solve, car contacts, integration in Bullet units and goal check
// (BallArena/Solve.cuh:56-117)
DI bool ballSleeping(const Dev& d, int sim)
{
    return lensq(d.sv(CARL_SIM_BALL_VEL, sim)) == 0.f && lensq(d.sv(CARL_SIM_BALL_ANG, sim)) == 0.f;
}

// solveArena(body, wasHit): the ball-arena solve at the exported ball
// position (not called when the ball sleeps).  Every word the tick tests is
// loaded in one batch before any test (the hit ticks and the near-car tests
// read car words that nothing before their use changes in this phase: the
// car-car pairs have run, and a car-ball pair writes only its own car); the
// ball's position and velocities then stay in registers through the car
// pairs and are stored once.
template <class SolveArena>
DI void ballTickWith(const Dev& d, int sim, int tick, SolveArena solveArena)
{
    const V3 ballVel = d.sv(CARL_SIM_BALL_VEL, sim), ballAng = d.sv(CARL_SIM_BALL_ANG, sim);
    const V3 exported = d.sv(CARL_SIM_BALL_POS, sim);
    const bool valid = d.si(CARL_SIM_BALL_INT_VALID, sim) != 0;
    const V3 expPos = d.sv(CARL_SIM_BALL_EXP_POS, sim), intPos = d.sv(CARL_SIM_BALL_INT_POS, sim);
    const V3 expVel = d.sv(CARL_SIM_BALL_EXP_VEL, sim), intVel = d.sv(CARL_SIM_BALL_INT_VEL, sim);
    const int base = sim * d.nCars;
    const V3 solverHalf{ kHalf.x + kCarMargin, kHalf.y + kCarMargin, kHalf.z + kCarMargin };
    const float maxDist = kBallRadius + len(solverHalf);
    bool hit = false;
    unsigned near = 0;
    for (int k = 0; k < d.nCars; k++) {
        const int h = d.ci(CARL_CAR_BALL_HIT_TICK, base + k);
        const bool demoed = d.ci(CARL_CAR_DEMOED, base + k) != 0;
        const V3 cen = d.cv(CARL_CAR_CEN, base + k);
        hit |= h >= 0 && tick > 0 && h == tick - 1;
        if (!demoed && !(lensq(exported - cen) > maxDist * maxDist)) near |= 1u << k;
    }
    const bool sleeping = lensq(ballVel) == 0.f && lensq(ballAng) == 0.f;
    V3 posBT = (valid && lensq(exported - expPos) == 0.f) ? intPos : exported * .02f;
    V3 velBT = (valid && lensq(ballVel - expVel) == 0.f) ? intVel : ballVel * .02f;
    const V3 damped = sleeping ? velBT : velBT * kBallDrag;
    const V3 preBT = sleeping ? velBT : damped + (kGravity * .02f) * kDt;
    const V3 velNoExt = damped * 50.f;
    const V3 preVel = preBT * 50.f;
    V3 pushVel = kZero;
    V3 pos = exported, vel = ballVel, ang = ballAng;
    if (!sleeping) {
        BallBody b;
        b.vel = preVel; b.velNoExt = velNoExt; b.ang = ballAng;
        b.dVel = kZero; b.dAng = kZero; b.pushVel = kZero; b.pushAng = kZero;
        solveArena(b, hit);
        vel = b.vel;
        ang = b.ang;
        pushVel = b.pushVel;
    }
    bool moved = !sleeping;
    for (int k = 0; k < d.nCars; k++)
        if (near & (1u << k)) moved |= ballCarPair(d, sim, base + k, preVel, tick, pos, vel, ang);
    if (moved) {
        d.ssetv(CARL_SIM_BALL_VEL, sim, vel);
        d.ssetv(CARL_SIM_BALL_ANG, sim, ang);
    }
    if (lensq(pos - exported) != 0.f) posBT = pos * .02f;
    velBT = lensq(vel - preVel) == 0.f ? preBT : vel * .02f;
    posBT = posBT + (pushVel * .02f) * kDt;
    posBT = posBT + velBT * kDt;
    const V3 ballPos = posBT * 50.f;
    d.ssetv(CARL_SIM_BALL_POS, sim, ballPos);
    d.ssetv(CARL_SIM_BALL_INT_POS, sim, posBT);
    d.ssetv(CARL_SIM_BALL_INT_VEL, sim, velBT);
    d.ssetv(CARL_SIM_BALL_EXP_POS, sim, ballPos);
    d.ssetv(CARL_SIM_BALL_EXP_VEL, sim, vel);
    d.sseti(CARL_SIM_BALL_INT_VALID, sim, 1);

    const float thr = kGoalThresholdY + kBallRadius;
    const int scorer = ballPos.y > thr ? 1 : (ballPos.y < -thr ? -1 : 0);
    if (!scorer || d.si(CARL_SIM_LAST_SCORER, sim) != 0) return;
    if (scorer > 0) d.sseti(CARL_SIM_BLUE_SCORE, sim, d.si(CARL_SIM_BLUE_SCORE, sim) + 1);
    else d.sseti(CARL_SIM_ORANGE_SCORE, sim, d.si(CARL_SIM_ORANGE_SCORE, sim) + 1);
    d.sseti(CARL_SIM_LAST_SCORER, sim, scorer);
    d.sseti(CARL_SIM_GOAL_TICK, sim, tick);
}

// cs/count: the arena contacts of the exported ball position (unused when
// the ball sleeps)
DI void ballTick(const Dev& d, int sim, int tick, const BallContact* cs, int count)
{
    ballTickWith(d, sim, tick, [&](BallBody& b, bool hit) { solveBallContacts(b, cs, count, hit); });
}

// the same with the native arena meshes
DI void nativeBallTick(const Dev& d, int sim, int tick)
{
    ballTickWith(d, sim, tick, [&](BallBody& b, bool hit) {
        const int n = gatherNativeBallContacts(d, sim, d.sv(CARL_SIM_BALL_POS, sim));
        solveNativeBallContacts(d, sim, b, n, hit);
    });
}

// ------------------------------------------------------------ finish, pads

DI void resetInternal(const Dev& d, int c)
{
    for (int f = CARL_CAR_ON_GROUND; f <= CARL_CAR_TIME_SINCE_BOOSTED; f++) d.seti(f, c, 0);
    d.seti(CARL_CAR_ON_GROUND, c, 1);
    d.setf(CARL_CAR_BOOST, c, kBoostSpawn);
}

DI void respawnCar(const Dev& d, int c)
{
    const int local = c % d.nCars;
    const int idx = d.ci(CARL_CAR_RESPAWN_IDX, c);
    const bool orange = local >= d.nBlue;
    const float y = orange ? -kRespawnY : kRespawnY;
    const float yaw = orange ? kRespawnYaw + kPi : kRespawnYaw;
    const Q4 rot = yawQuat(yaw);
    const V3 pos{ respawnX(idx), y, kCarRespawnZ };
    d.setv(CARL_CAR_POS, c, pos);
    d.setv(CARL_CAR_CEN, c, pos + rotate(rot, kHitboxOffset));
    d.setq(CARL_CAR_ROT, c, rot);
    d.setv(CARL_CAR_VEL, c, kZero);
    d.setv(CARL_CAR_ANG, c, kZero);
    d.setv(CARL_CAR_IMP, c, kZero);
    d.seti(CARL_CAR_DEMOED, c, 0);
    d.setf(CARL_CAR_DEMO_TIMER, c, 0.f);
    d.seti(CARL_CAR_CONTACT_IDX, c, -1);
    d.setf(CARL_CAR_CONTACT_COOLDOWN, c, 0.f);
    d.seti(CARL_CAR_BALL_HIT_TICK, c, -1);
    d.seti(CARL_CAR_BALL_CONTACT_TICK, c, -1);
    for (int k = 0; k < kWheels; k++) d.seti(CARL_CAR_WHEEL_CONTACT + k, c, 0);
    resetInternal(d, c);
}

// integrate, then apply the impulse cache / demo timer (Solve.cuh:316-327, FinishTick.cuh:100-141)
DI void finishCar(const Dev& d, int c)
{
    V3 pos = d.cv(CARL_CAR_POS, c), cen;
    Q4 rot = d.cq(CARL_CAR_ROT, c);
    V3 vel = d.cv(CARL_CAR_VEL, c), ang = d.cv(CARL_CAR_ANG, c);
    const V3 imp = d.cv(CARL_CAR_IMP, c);
    const float cd = d.cf(CARL_CAR_CONTACT_COOLDOWN, c);
    if (d.ci(CARL_CAR_DEMOED, c)) {
        float timer = d.cf(CARL_CAR_DEMO_TIMER, c);
        if (timer <= kDemoRespawnTime) {
            const float st = d.cf(CARL_CAR_CTRL_STEER, c);
            const int dir = st < -kDemoInputDeadzone ? -1 : (st > kDemoInputDeadzone ? 1 : 0);
            const int lastDir = d.ci(CARL_CAR_LAST_RESPAWN_DIR, c);
            if (dir != 0 && dir != lastDir) {
                const int idx = d.ci(CARL_CAR_RESPAWN_IDX, c);
                if (dir < 0 && idx > 0) d.seti(CARL_CAR_RESPAWN_IDX, c, idx - 1);
                else if (dir > 0 && idx < 3) d.seti(CARL_CAR_RESPAWN_IDX, c, idx + 1);
            }
            d.seti(CARL_CAR_LAST_RESPAWN_DIR, c, dir);
        }
        timer = fmax_(timer - kDt, 0.f);
        d.setf(CARL_CAR_DEMO_TIMER, c, timer);
        if (timer <= 0.f) respawnCar(d, c);
        return;
    }
    integratePose(pos, cen, rot, vel, ang);
    clampCarVelocity(vel, ang);
    if (lensq(imp) > 1e-12f) {
        vel = vel + imp;
        const float ss = lensq(vel);
        if (ss > kCarMaxSpeed * kCarMaxSpeed) vel = vel * (kCarMaxSpeed * rsqrt_(ss));
        d.setv(CARL_CAR_IMP, c, kZero);
    }
    d.setv(CARL_CAR_POS, c, pos);
    d.setv(CARL_CAR_CEN, c, cen);
    d.setq(CARL_CAR_ROT, c, rot);
    d.setv(CARL_CAR_VEL, c, vel);
    d.setv(CARL_CAR_ANG, c, ang);
    if (cd > 0.f) d.setf(CARL_CAR_CONTACT_COOLDOWN, c, fmax_(cd - kDt, 0.f));
}

DI void finishBall(const Dev& d, int s)
{
    V3 vel = d.sv(CARL_SIM_BALL_VEL, s) + d.sv(CARL_SIM_BALL_IMP, s);
    V3 ang = d.sv(CARL_SIM_BALL_ANG, s);
    float ss = lensq(vel);
    if (ss > kBallMaxSpeed * kBallMaxSpeed) vel = vel * (kBallMaxSpeed * rsqrt_(ss));
    ss = lensq(ang);
    if (ss > kBallMaxAng * kBallMaxAng) ang = ang * (kBallMaxAng * rsqrt_(ss));
    d.ssetv(CARL_SIM_BALL_VEL, s, vel);
    d.ssetv(CARL_SIM_BALL_ANG, s, ang);
    d.ssetv(CARL_SIM_BALL_IMP, s, kZero);
}

// pads of one simulation, in pad order; the last overlapping car takes the pad.
// The cars' positions, demo flags and boost live in registers for the whole
// pass (at most MaxCars per simulation, the loops over them unrolled);
// boosts are written back once.  The pass is instantiated for two, four and
// eight cars, so that 1v1 runs a quarter of the 8-car code (measured 3% per
// step on the 1v1 window kernel).
constexpr int kMaxCars = 8;

// Boost pads [p0, p1) of simulation s: cooldowns, pickups and the boost
// they give.  No car position lies in two pads' cylinders (the closest pair
// of cylinders is 773 uu apart), so a car takes boost from at most one pad per
// tick: disjoint pad ranges of one simulation can run in different threads,
// in any order, with the same result.  A thread reads every car's boost but
// uses it only for a car inside one of its own pads, the only case in which
// it writes that boost.  [P0, P1) bounds the range at compile time (a
// caller whose range is fixed loads only those pads' cooldowns).
template <int MaxCars, int P0 = 0, int P1 = kPads>
DI void boostPadsRangeT(const Dev& d, int s, int p0, int p1)
{
    const int base = s * d.nCars;
    V3 cp[MaxCars];
    bool alive[MaxCars];
    float boost[MaxCars];
#pragma unroll
    for (int k = 0; k < MaxCars; k++) {
        alive[k] = false;
        cp[k] = kZero;
        boost[k] = 0.f;
        if (k < d.nCars) {
            alive[k] = !d.ci(CARL_CAR_DEMOED, base + k);
            cp[k] = d.cv(CARL_CAR_POS, base + k);
            boost[k] = d.cf(CARL_CAR_BOOST, base + k);
        }
    }
    // all cooldowns are read before any is written back, each load
    // unconditional (one batch in flight; a load under a per-pad range test
    // would wait for its own round trip), those outside the range unused
    float cool[kPads];
#pragma unroll
    for (int p = P0; p < P1; p++) cool[p] = d.sf(CARL_SIM_PAD_COOLDOWN + p, s);
    int changed = 0;
#pragma unroll
    for (int p = P0; p < P1; p++) {
        if (p < p0 || p >= p1) continue;
        const float prev = cool[p];
        float cd = prev;
        if (cd > 0.f) cd = fmax_(cd - kDt, 0.f);
        if (cd <= 0.f) {
            const bool big = p < 6;
            const float radius = big ? kBigPadRadius : kSmallPadRadius;
            const float px = kPadPos[p][0], py = kPadPos[p][1], pz = kPadPos[p][2];
            int locked = -1;
            float have = 0.f;
#pragma unroll
            for (int k = 0; k < MaxCars; k++) {
                if (k >= d.nCars || !alive[k]) continue;
                const float dx = cp[k].x - px, dy = cp[k].y - py;
                if (dx * dx + dy * dy < radius * radius && fabsf(cp[k].z - pz) < kPadHeight) {
                    locked = k;
                    have = boost[k];
                }
            }
            if (locked >= 0 && have < kBoostMax) {
                const float next = fmin_(have + (big ? kBigPadAmount : kSmallPadAmount), kBoostMax);
                setAt(boost, locked, next);
                changed |= 1 << locked;
                cd = big ? kBigPadCooldown : kSmallPadCooldown;
            }
        }
        if (__float_as_uint(cd) != __float_as_uint(prev)) d.ssetf(CARL_SIM_PAD_COOLDOWN + p, s, cd);
    }
#pragma unroll
    for (int k = 0; k < MaxCars; k++)
        if (changed & (1 << k)) d.setf(CARL_CAR_BOOST, base + k, boost[k]);
}

// The same for a range of at most Span pads whose bounds vary from lane to
// lane (the workgroup's pad parts do not line up with its waves): the pads
// are visited as positions p0 + i, i < Span, so every lane runs the same
// iterations, with the pads' positions read from the table by index; only
// the range's cooldowns are loaded (all before the first is used).
template <int MaxCars, int Span>
DI void boostPadsSpanT(const Dev& d, int s, int p0, int p1)
{
    const int base = s * d.nCars;
    V3 cp[MaxCars];
    bool alive[MaxCars];
    float boost[MaxCars];
#pragma unroll
    for (int k = 0; k < MaxCars; k++) {
        alive[k] = false;
        cp[k] = kZero;
        boost[k] = 0.f;
        if (k < d.nCars) {
            alive[k] = !d.ci(CARL_CAR_DEMOED, base + k);
            cp[k] = d.cv(CARL_CAR_POS, base + k);
            boost[k] = d.cf(CARL_CAR_BOOST, base + k);
        }
    }
    float cool[Span];
#pragma unroll
    for (int i = 0; i < Span; i++) cool[i] = d.sf(CARL_SIM_PAD_COOLDOWN + min(p0 + i, kPads - 1), s);
    int changed = 0;
#pragma unroll
    for (int i = 0; i < Span; i++) {
        const int p = p0 + i;
        if (p >= p1) break;
        const float prev = cool[i];
        float cd = prev;
        if (cd > 0.f) cd = fmax_(cd - kDt, 0.f);
        if (cd <= 0.f) {
            const bool big = p < 6;
            const float radius = big ? kBigPadRadius : kSmallPadRadius;
            const float px = kPadPos[p][0], py = kPadPos[p][1], pz = kPadPos[p][2];
            int locked = -1;
            float have = 0.f;
#pragma unroll
            for (int k = 0; k < MaxCars; k++) {
                if (k >= d.nCars || !alive[k]) continue;
                const float dx = cp[k].x - px, dy = cp[k].y - py;
                if (dx * dx + dy * dy < radius * radius && fabsf(cp[k].z - pz) < kPadHeight) {
                    locked = k;
                    have = boost[k];
                }
            }
            if (locked >= 0 && have < kBoostMax) {
                const float next = fmin_(have + (big ? kBigPadAmount : kSmallPadAmount), kBoostMax);
                setAt(boost, locked, next);
                changed |= 1 << locked;
                cd = big ? kBigPadCooldown : kSmallPadCooldown;
            }
        }
        if (__float_as_uint(cd) != __float_as_uint(prev)) d.ssetf(CARL_SIM_PAD_COOLDOWN + p, s, cd);
    }
#pragma unroll
    for (int k = 0; k < MaxCars; k++)
        if (changed & (1 << k)) d.setf(CARL_CAR_BOOST, base + k, boost[k]);
}

// pads [p0, p1) of simulation s, the range at most ceil(kPads / parts) long
DI void boostPadsSpan(const Dev& d, int s, int p0, int p1, int parts)
{
    const int span = (kPads + parts - 1) / parts;
    if (d.nCars <= 2) {
        if (span <= 3) boostPadsSpanT<2, 3>(d, s, p0, p1);
        else if (span <= 9) boostPadsSpanT<2, 9>(d, s, p0, p1);
        else if (span <= kPads / 2) boostPadsSpanT<2, kPads / 2>(d, s, p0, p1);
        else boostPadsSpanT<2, kPads>(d, s, p0, p1);
    } else if (d.nCars <= 4) {
        if (span <= 3) boostPadsSpanT<4, 3>(d, s, p0, p1);
        else if (span <= 9) boostPadsSpanT<4, 9>(d, s, p0, p1);
        else boostPadsSpanT<4, kPads>(d, s, p0, p1);
    } else {
        if (span <= 6) boostPadsSpanT<kMaxCars, 6>(d, s, p0, p1);
        else boostPadsSpanT<kMaxCars, kPads>(d, s, p0, p1);
    }
}

DI void boostPadsRange(const Dev& d, int s, int p0, int p1)
{
    if (d.nCars <= 2) boostPadsRangeT<2>(d, s, p0, p1);
    else if (d.nCars <= 4) boostPadsRangeT<4>(d, s, p0, p1);
    else boostPadsRangeT<kMaxCars>(d, s, p0, p1);
}

DI void boostPads(const Dev& d, int s) { boostPadsRange(d, s, 0, kPads); }

}  // namespace carl
