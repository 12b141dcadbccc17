// envio.h - observation / state / reward packing, resets and state setters.
//
// Reference semantics:
//   observation layout and orange mirroring   include/Physics/Observations.cuh:9-238
//   normalisation                             include/Physics/Observations.cuh:240-317
//   canonical state                           include/Physics/Observations.cuh:320-356
//   rewards, dones, overtime                  include/Physics/Observations.cuh:360-397
//   kickoff / done resets                     include/State/Reset.cuh:8-171
//   full reset                                include/State/GameState.cuh:221-231,
//                                             include/State/Workspace.cuh:225-233
//   setters and contact refresh               src/EnvIO.cu:137-357, 603-643
#pragma once

#include "sim_phase.h"

namespace carl {

DI V3 mirrorXY(V3 v, bool inv) { return inv ? V3{ -v.x, -v.y, v.z } : v; }

DI void put3(float* o, int& k, V3 v)
{
    o[k++] = v.x;
    o[k++] = v.y;
    o[k++] = v.z;
}

DI void packCar(const Dev& d, int c, bool inv, float* o, int& k)
{
    const Q4 rot = d.cq(CARL_CAR_ROT, c);
    put3(o, k, mirrorXY(d.cv(CARL_CAR_POS, c), inv));
    put3(o, k, mirrorXY(d.cv(CARL_CAR_VEL, c), inv));
    put3(o, k, mirrorXY(d.cv(CARL_CAR_ANG, c), inv));
    put3(o, k, mirrorXY(rotate(rot, kX), inv));
    put3(o, k, mirrorXY(rotate(rot, kZ), inv));
    o[k++] = d.cf(CARL_CAR_BOOST, c);
    o[k++] = (float)d.ci(CARL_CAR_ON_GROUND, c);
    o[k++] = (float)(d.ci(CARL_CAR_DEMOED, c) != 0);
    o[k++] = (float)d.ci(CARL_CAR_HAS_FLIPPED, c);
    o[k++] = (float)d.ci(CARL_CAR_HAS_DOUBLE_JUMPED, c);
    o[k++] = (float)d.ci(CARL_CAR_IS_BOOSTING, c);
}

// Rows are built in kRowParts column parts, one lane per part, so that the
// four waves of a packing workgroup share every row's arithmetic.
constexpr int kRowParts = 4;

// Column of the first pad flag in an observation row (pad distances follow
// the kPads flags).
HDI int obsPadColumn(int nCars) { return 9 + nCars * kObsPerCar; }

// Pad columns of part Part > 0 of one observer's row: the flag and the
// distance of the pads p = Part - 1, Part + 2, ... (p % 3 == Part - 1).  The
// part is a template argument, so every pad index, its table position and its
// mirrored index are compile-time constants: the positions fold into
// immediates and no load waits on another.  An orange observer's slot p shows
// pad mirroredPad(p), which sits at pad p's position with x and y negated
// (the table is symmetric through the field centre); its cooldown field is
// chosen per lane inside the load's offset.
template <int Part>
DI void packObservationPads(const Dev& d, int sim, bool inv, bool normalizeObs, V3 egoPos, int padCol, float* o)
{
    constexpr int kMine = (kPads - (Part - 1) + 2) / 3;
    const float sgn = inv ? -1.f : 1.f;
    float cool[kMine];
#pragma unroll
    for (int i = 0; i < kMine; i++) {
        const int p = Part - 1 + 3 * i;
        cool[i] = __uint_as_float(d.swLane(CARL_SIM_PAD_COOLDOWN + (inv ? mirroredPad(p) : p), sim));
    }
#pragma unroll
    for (int i = 0; i < kMine; i++) {
        const int p = Part - 1 + 3 * i;
        o[padCol + p] = cool[i] <= 0.f;
        const float dist = len(egoPos - V3{ kPadPos[p][0] * sgn, kPadPos[p][1] * sgn, kPadPos[p][2] });
        o[padCol + kPads + p] = normalizeObs ? dist / 14692.54f : dist;
    }
}

// Car `c` of the simulation, the j-th other car of observer `obs` in
// observation order: its teammates (without itself), then its opponents.
DI int otherCar(const Dev& d, int obs, int j)
{
    const bool orange = obs >= d.nBlue;
    const int tS = orange ? d.nBlue : 0, tE = orange ? d.nCars : d.nBlue;
    const int oS = orange ? 0 : d.nBlue;
    const int mates = tE - tS - 1;
    if (j < mates) return tS + j + (tS + j >= obs ? 1 : 0);
    return oS + (j - mates);
}

constexpr float kObsScaleX = 4108.f, kObsScaleY = 6000.f, kObsScaleZ = 2076.f;

// The columns of other cars j0, j0 + step, ... of one observer: each one's
// car block and its position and velocity relative to the observer.
DI void packObservationOthers(const Dev& d, int sim, int obs, bool inv, bool normalizeObs, int j0, int step,
                              V3 egoPos, V3 egoVel, float* o)
{
    const int nC = d.nCars, base = sim * nC;
    const V3 scale{ kObsScaleX, kObsScaleY, kObsScaleZ };
    const int relCol = obsPadColumn(nC) + 2 * kPads + 6;
    for (int j = j0; j < nC - 1; j += step) {
        const int c = base + otherCar(d, obs, j);
        int k = 9 + (1 + j) * kObsPerCar;
        packCar(d, c, inv, o, k);
        int r = relCol + 6 * j;
        put3(o, r, mirrorXY(d.cv(CARL_CAR_POS, c) - egoPos, inv));
        put3(o, r, mirrorXY(d.cv(CARL_CAR_VEL, c) - egoVel, inv));
        if (!normalizeObs) continue;
        const int off = 9 + (1 + j) * kObsPerCar;
        for (int a = 0; a < 3; a++) o[off + a] /= comp(scale, a);
        for (int a = 3; a < 6; a++) o[off + a] /= kCarMaxSpeed;
        for (int a = 6; a < 9; a++) o[off + a] /= kCarMaxAng;
        o[off + 15] /= kBoostMax;
        r = relCol + 6 * j;
        for (int a = 0; a < 3; a++) {
            o[r + a] /= 2.f * comp(scale, a);
            o[r + 3 + a] /= 2.f * kCarMaxSpeed;
        }
    }
}

// Part `part` of one observer's row: ball, self, teammates, opponents, pads,
// relative vectors, goals, dodge window, controller state [, previous
// controls].  Part 0 writes the ball's and the observer's own columns, part
// q > 0 the flag and the distance of the pads p with p % 3 == q - 1; the
// other cars' columns go to part 0 in 1v1 (one other car: measured faster
// there) and, with more cars, to part q for the other cars j with
// j % 3 == q - 1 (2v2 packing 173 -> 155 us, 3v3 92 -> 75 us).  Each part
// normalises its own columns.
DI void packObservationPart(const Dev& d, int sim, int obs, bool invertOrange, bool normalizeObs, bool prev, int part,
                            float* o)
{
    const int nC = d.nCars, base = sim * nC;
    const bool orange = obs >= d.nBlue;
    const bool inv = invertOrange && orange;
    const int ego = base + obs;
    const V3 egoPos = d.cv(CARL_CAR_POS, ego);
    const V3 egoVel = d.cv(CARL_CAR_VEL, ego);
    const int padCol = obsPadColumn(nC);
    static_assert(kRowParts == 4, "three pad parts");
    const bool spread = nC > 2;
    if (part > 0) {
        if (spread) packObservationOthers(d, sim, obs, inv, normalizeObs, part - 1, kRowParts - 1, egoPos, egoVel, o);
        switch (part) {
        case 1: packObservationPads<1>(d, sim, inv, normalizeObs, egoPos, padCol, o); return;
        case 2: packObservationPads<2>(d, sim, inv, normalizeObs, egoPos, padCol, o); return;
        default: packObservationPads<3>(d, sim, inv, normalizeObs, egoPos, padCol, o); return;
        }
    }
    const V3 ballPos = d.sv(CARL_SIM_BALL_POS, sim), ballVel = d.sv(CARL_SIM_BALL_VEL, sim);
    int k = 0;
    put3(o, k, mirrorXY(ballPos, inv));
    put3(o, k, mirrorXY(ballVel, inv));
    put3(o, k, mirrorXY(d.sv(CARL_SIM_BALL_ANG, sim), inv));
    packCar(d, ego, inv, o, k);
    if (!spread) packObservationOthers(d, sim, obs, inv, normalizeObs, 0, 1, egoPos, egoVel, o);
    k = padCol + 2 * kPads;
    put3(o, k, mirrorXY(ballPos - egoPos, inv));
    put3(o, k, mirrorXY(ballVel - egoVel, inv));
    k += 6 * (nC - 1);
    const float ownY = orange ? kGoalCenterY : -kGoalCenterY;
    put3(o, k, mirrorXY(V3{ 0.f, ownY, kGoalCenterZ } - ballPos, inv));
    put3(o, k, mirrorXY(V3{ 0.f, -ownY, kGoalCenterZ } - ballPos, inv));
    const float atsj = d.cf(CARL_CAR_AIR_TIME_SINCE_JUMP, ego);
    const bool flip = !d.ci(CARL_CAR_HAS_FLIPPED, ego) && !d.ci(CARL_CAR_HAS_DOUBLE_JUMPED, ego) && atsj < kDoubleJumpWindow;
    o[k++] = (float)flip;
    o[k++] = flip ? fmax_(0.f, kDoubleJumpWindow - atsj) : 0.f;
    o[k++] = (float)d.ci(CARL_CAR_HAS_JUMPED, ego);
    o[k++] = (float)d.ci(CARL_CAR_IS_JUMPING, ego);
    o[k++] = (float)d.ci(CARL_CAR_IS_FLIPPING, ego);
    o[k++] = d.cf(CARL_CAR_FLIP_TIME, ego);
    o[k++] = d.cf(CARL_CAR_DEMO_TIMER, ego);
    if (prev) {
        o[k++] = d.cf(CARL_CAR_CTRL_THROTTLE, ego);
        o[k++] = d.cf(CARL_CAR_CTRL_STEER, ego);
        o[k++] = d.cf(CARL_CAR_CTRL_YAW, ego);
        o[k++] = d.cf(CARL_CAR_CTRL_PITCH, ego);
        o[k++] = d.cf(CARL_CAR_CTRL_ROLL, ego);
        o[k++] = (float)d.ci(CARL_CAR_CTRL_JUMP, ego);
        o[k++] = (float)d.ci(CARL_CAR_CTRL_BOOST, ego);
        o[k++] = (float)d.ci(CARL_CAR_CTRL_SLIDE, ego);
    }
    if (!normalizeObs) return;
    const V3 scale{ kObsScaleX, kObsScaleY, kObsScaleZ };
    for (int a = 0; a < 3; a++) o[a] /= comp(scale, a);
    for (int a = 3; a < 6; a++) o[a] /= kBallMaxSpeed;
    for (int a = 6; a < 9; a++) o[a] /= kBallMaxAng;
    {
        const int off = 9;
        for (int a = 0; a < 3; a++) o[off + a] /= comp(scale, a);
        for (int a = 3; a < 6; a++) o[off + a] /= kCarMaxSpeed;
        for (int a = 6; a < 9; a++) o[off + a] /= kCarMaxAng;
        o[off + 15] /= kBoostMax;
    }
    int r = padCol + 2 * kPads;
    for (int a = 0; a < 3; a++) {
        o[r + a] /= 2.f * comp(scale, a);
        o[r + 3 + a] /= kBallMaxSpeed + kCarMaxSpeed;
    }
    r += 6 + 6 * (nC - 1);
    for (int g = 0; g < 2; g++)
        for (int a = 0; a < 3; a++) o[r + g * 3 + a] /= 2.f * comp(scale, a);
}

// Part `part` of a simulation's canonical state row (ball, cars, pad flags):
// part 0 writes the ball and the pad flags, part q > 0 the cars c with
// c % 3 == q - 1.
DI void packStatePart(const Dev& d, int sim, int touchWindow, int tickCount, int part, float* o)
{
    if (part == 0) {
        int k = 0;
        put3(o, k, d.sv(CARL_SIM_BALL_POS, sim));
        put3(o, k, d.sv(CARL_SIM_BALL_VEL, sim));
        put3(o, k, d.sv(CARL_SIM_BALL_ANG, sim));
        k = 9 + d.nCars * kStatePerCar;
        for (int p = 0; p < kPads; p++) o[k++] = d.sf(CARL_SIM_PAD_COOLDOWN + p, sim) <= 0.f;
        return;
    }
    for (int c = part - 1; c < d.nCars; c += 3) {
        const int car = sim * d.nCars + c;
        int k = 9 + c * kStatePerCar;
        packCar(d, car, false, o, k);
        o[k++] = d.ci(CARL_CAR_BALL_CONTACT_TICK, car) > tickCount - touchWindow;
    }
}

struct DoneRule {
    int maxTicks, overtimeTicks, noTouchTicks;
};

// The match words that decide whether an episode ends.
struct MatchWords {
    int ep, blue, orange, overtime, scorer, lastTouch;
};

DI MatchWords matchWords(const Dev& d, int s)
{
    return MatchWords{ d.si(CARL_SIM_EPISODE_TICKS, s), d.si(CARL_SIM_BLUE_SCORE, s), d.si(CARL_SIM_ORANGE_SCORE, s),
                       d.si(CARL_SIM_OVERTIME, s),      d.si(CARL_SIM_LAST_SCORER, s), d.si(CARL_SIM_LAST_TOUCH_TICK, s) };
}

DI bool simDoneFrom(const MatchWords& m, int tickCount, DoneRule rule)
{
    const bool overtime = m.overtime != 0;
    const bool regExpired = m.ep >= rule.maxTicks && m.blue != m.orange;
    const bool otExpired = overtime && m.ep >= rule.maxTicks + rule.overtimeTicks;
    const bool scored = m.scorer != 0;
    const bool timeout = rule.noTouchTicks > 0 && tickCount - m.lastTouch >= rule.noTouchTicks;
    return (!overtime && regExpired) || otExpired || timeout || scored;
}

DI bool simDone(const Dev& d, int s, int tickCount, DoneRule rule)
{
    return simDoneFrom(matchWords(d, s), tickCount, rule);
}

// ------------------------------------------------------------------ resets

DI void kickoffCar(const Dev& d, int c, int loc, bool invert)
{
    const int l = loc % 5;
    const float x = invert ? -kickoffX(l) : kickoffX(l);
    const float y = invert ? -kickoffY(l) : kickoffY(l);
    const float yaw = invert ? kickoffYaw(l) + kPi : kickoffYaw(l);
    const V3 pos{ x, y, kCarRestZ };
    const Q4 rot = yawQuat(yaw);
    d.setv(CARL_CAR_POS, c, pos);
    d.setv(CARL_CAR_VEL, c, kZero);
    d.setv(CARL_CAR_ANG, c, kZero);
    d.setq(CARL_CAR_ROT, c, rot);
    d.setv(CARL_CAR_CEN, c, pos + rotate(rot, kHitboxOffset));
    d.setv(CARL_CAR_IMP, c, kZero);
    d.seti(CARL_CAR_DEMOED, c, 0);
    d.setf(CARL_CAR_DEMO_TIMER, c, 0.f);
    d.seti(CARL_CAR_CONTACT_IDX, c, -1);
    d.setf(CARL_CAR_CONTACT_COOLDOWN, c, 0.f);
    d.seti(CARL_CAR_BALL_HIT_TICK, c, -1);
    d.seti(CARL_CAR_BALL_CONTACT_TICK, c, -1);
    for (int f = CARL_CAR_CTRL_THROTTLE; f <= CARL_CAR_CTRL_SLIDE; f++) d.seti(f, c, 0);
    for (int k = 0; k < kWheels; k++) d.seti(CARL_CAR_WHEEL_CONTACT + k, c, 0);
    resetInternal(d, c);
}

// The kickoff permutation of simulation s after a reset at tickCount.
DI int kickoffPerm(const Dev& d, int s, int tickCount)
{
    const uint32_t seed = mix32((uint32_t)d.seed) ^ mix32((uint32_t)s) ^ mix32((uint32_t)tickCount);
    return pickIndex(seed, 120);
}

DI void kickoffBall(const Dev& d, int s)
{
    d.ssetv(CARL_SIM_BALL_POS, s, V3{ 0.f, 0.f, kBallRestZ });
    d.ssetv(CARL_SIM_BALL_VEL, s, kZero);
    d.ssetv(CARL_SIM_BALL_ANG, s, kZero);
    d.sseti(CARL_SIM_BALL_INT_VALID, s, 0);
}

// Car `local` of simulation s at its kickoff spawn (blue cars first, then
// orange, each team numbered from 0 in the permutation).
DI void kickoffLocalCar(const Dev& d, int s, int local, int perm)
{
    const bool orange = local >= d.nBlue;
    kickoffCar(d, s * d.nCars + local, kickoffSpawn(perm, orange ? local - d.nBlue : local), orange);
}

DI void kickoffSim(const Dev& d, int s, int tickCount, int nOrange)
{
    const int perm = kickoffPerm(d, s, tickCount);
    kickoffBall(d, s);
    for (int k = 0; k < d.nBlue + nOrange; k++) kickoffLocalCar(d, s, k, perm);
}

DI void clearCarContacts(const Dev& d, int c)
{
    d.setf(CARL_CAR_BRAKE_STAGE, c, 0.f);
    d.setf(CARL_CAR_STEER_STAGE, c, 0.f);
    d.setf(CARL_CAR_DRIVE_STAGE, c, 0.f);
    d.seti(CARL_CAR_MANIFOLD_COUNT, c, 0);
    for (int k = 0; k < kWheels; k++) {
        d.setf(CARL_CAR_LAT_FRICTION + k, c, 0.f);
        d.setf(CARL_CAR_LON_FRICTION + k, c, 0.f);
    }
}

DI void fullResetSim(const Dev& d, int s, int nOrange)
{
    d.sseti(CARL_SIM_EPISODE_TICKS, s, 0);
    d.sseti(CARL_SIM_LAST_TOUCH_TICK, s, 0);
    d.ssetv(CARL_SIM_BALL_IMP, s, kZero);
    d.sseti(CARL_SIM_BALL_INT_VALID, s, 0);
    for (int p = 0; p < kPads; p++) d.ssetf(CARL_SIM_PAD_COOLDOWN + p, s, 0.f);
    for (int f = CARL_SIM_BLUE_SCORE; f <= CARL_SIM_OVERTIME; f++) d.sseti(f, s, 0);
    d.sseti(CARL_SIM_BALL_ARENA_CONTACT_TICK, s, -1);
    for (int k = 0; k < d.nCars; k++) {
        const int c = s * d.nCars + k;
        d.setv(CARL_CAR_IMP, c, kZero);
        d.seti(CARL_CAR_DEMOED, c, 0);
        d.setf(CARL_CAR_DEMO_TIMER, c, 0.f);
        d.seti(CARL_CAR_CONTACT_IDX, c, -1);
        d.setf(CARL_CAR_CONTACT_COOLDOWN, c, 0.f);
        d.seti(CARL_CAR_BALL_HIT_TICK, c, -1);
        d.seti(CARL_CAR_BALL_CONTACT_TICK, c, -1);
        for (int w = 0; w < kWheels; w++) {
            d.seti(CARL_CAR_WHEEL_SOURCE + w, c, kSrcNone);
            d.seti(CARL_CAR_WHEEL_CONTACT + w, c, 0);
        }
        d.seti(CARL_CAR_ARENA_CONTACT_TICK, c, -1);
        resetInternal(d, c);
        clearCarContacts(d, c);
    }
    kickoffSim(d, s, 0, nOrange);
}

// What the end-of-step reset does to one simulation: nothing, enter
// overtime (a tie at the end of regulation), or reset it to a kickoff.
enum DoneOutcome { kKept = 0, kOvertimeEntered = 1, kReset = 2 };

DI int doneOutcome(const MatchWords& m, int tickCount, DoneRule rule)
{
    const bool scored = m.scorer != 0;
    const bool overtime = m.overtime != 0;
    const bool noTouch = rule.noTouchTicks > 0 && tickCount - m.lastTouch >= rule.noTouchTicks;
    const bool otExpired = overtime && m.ep >= rule.maxTicks + rule.overtimeTicks;
    const bool timeout = m.ep >= rule.maxTicks;
    if (!overtime && !scored && !noTouch && m.ep >= rule.maxTicks && m.blue == m.orange) return kOvertimeEntered;
    if (!(scored || noTouch || otExpired || (!overtime && timeout))) return kKept;
    return kReset;
}

// The car words a done-reset writes for car `local` of simulation s.
DI void resetCarAfterDone(const Dev& d, int s, int local, int perm)
{
    const int c = s * d.nCars + local;
    kickoffLocalCar(d, s, local, perm);
    d.seti(CARL_CAR_ARENA_CONTACT_TICK, c, -1);
    clearCarContacts(d, c);
    for (int w = 0; w < kWheels; w++) {
        d.seti(CARL_CAR_WHEEL_SOURCE + w, c, kSrcNone);
        d.seti(CARL_CAR_WHEEL_CONTACT + w, c, 0);
    }
}

// The simulation words (match state, clock, ball) a done-reset writes.
DI void resetSimWordsAfterDone(const Dev& d, int s, int tickCount)
{
    for (int f = CARL_SIM_BLUE_SCORE; f <= CARL_SIM_OVERTIME; f++) d.sseti(f, s, 0);
    kickoffBall(d, s);
    d.sseti(CARL_SIM_EPISODE_TICKS, s, 0);
    d.sseti(CARL_SIM_LAST_TOUCH_TICK, s, tickCount);
    d.sseti(CARL_SIM_BALL_ARENA_CONTACT_TICK, s, -1);
}

DI void applyDoneOutcome(const Dev& d, int s, int outcome, int tickCount, int nOrange)
{
    if (outcome == kOvertimeEntered) {
        d.sseti(CARL_SIM_OVERTIME, s, 1);
        return;
    }
    if (outcome != kReset) return;
    const int perm = kickoffPerm(d, s, tickCount);
    resetSimWordsAfterDone(d, s, tickCount);
    for (int k = 0; k < d.nBlue + nOrange; k++) resetCarAfterDone(d, s, k, perm);
    for (int p = 0; p < kPads; p++) d.ssetf(CARL_SIM_PAD_COOLDOWN + p, s, 0.f);
}

// applyDoneOutcome shared by the kRowParts waves of a workgroup, each storing
// its own fields: wave 0 the simulation words, wave 1 the pad cooldowns,
// waves 2 and 3 the cars (car k by wave 2 + k % 2).  The waves write
// disjoint words, so the result is the same as one wave's.
DI void applyDoneOutcomePart(const Dev& d, int s, int outcome, int tickCount, int nOrange, int part)
{
    static_assert(kRowParts == 4, "four reset parts");
    if (outcome == kOvertimeEntered) {
        if (part == 0) d.sseti(CARL_SIM_OVERTIME, s, 1);
        return;
    }
    if (outcome != kReset) return;
    if (part == 0) {
        resetSimWordsAfterDone(d, s, tickCount);
    } else if (part == 1) {
        for (int p = 0; p < kPads; p++) d.ssetf(CARL_SIM_PAD_COOLDOWN + p, s, 0.f);
    } else {
        const int perm = kickoffPerm(d, s, tickCount);
        for (int k = part - 2; k < d.nBlue + nOrange; k += 2) resetCarAfterDone(d, s, k, perm);
    }
}

DI void resetAfterDone(const Dev& d, int s, int tickCount, DoneRule rule, int nOrange)
{
    applyDoneOutcome(d, s, doneOutcome(matchWords(d, s), tickCount, rule), tickCount, nOrange);
}

// ----------------------------------------------------------------- setters

// Input rows r < n, each targeting simulation indices[r] (r without
// indices); with a mask only the rows it sets.  A masked selection may also
// name its rows in a compacted list (ascending rows, list[0..*count) on the
// device), so that the setters and the repacking run over the selected rows
// only.
struct Selection {
    const int64_t* indices;
    const uint8_t* mask;
    int n;
    const int* list;
    const int* count;
};

// the input row handled by work item i, or -1 past the selection
DI int selectedInput(const Selection& sel, int i)
{
    if (sel.list) return i < *sel.count ? sel.list[i] : -1;
    return i < sel.n ? i : -1;
}

// target simulation of input row r, or -1 when the row is skipped
DI int selectRow(const Selection& sel, int r, int nSim)
{
    if (sel.mask && !sel.mask[r]) return -1;
    const int64_t t = sel.indices ? sel.indices[r] : r;
    return (t < 0 || t >= nSim) ? -1 : (int)t;
}

DI void setCarRow(const Dev& d, int src, int target, int local, const float* pos, const float* rot, const float* vel,
                  const float* ang, const void* demoed, bool byteDemoed, const float* boost, const float* internal)
{
    const int c = target * d.nCars + local;
    const float prevBoost = d.cf(CARL_CAR_BOOST, c);
    const int dm = byteDemoed ? (int)((const uint8_t*)demoed)[src] : ((const int32_t*)demoed)[src];
    const V3 p{ pos[3 * src], pos[3 * src + 1], pos[3 * src + 2] };
    const Q4 q{ rot[4 * src], rot[4 * src + 1], rot[4 * src + 2], rot[4 * src + 3] };
    d.setv(CARL_CAR_POS, c, p);
    d.setq(CARL_CAR_ROT, c, q);
    d.setv(CARL_CAR_VEL, c, V3{ vel[3 * src], vel[3 * src + 1], vel[3 * src + 2] });
    d.setv(CARL_CAR_ANG, c, V3{ ang[3 * src], ang[3 * src + 1], ang[3 * src + 2] });
    d.setv(CARL_CAR_CEN, c, p + rotate(q, kHitboxOffset));
    d.setv(CARL_CAR_IMP, c, kZero);
    d.seti(CARL_CAR_DEMOED, c, dm != 0 ? 1 : 0);
    d.setf(CARL_CAR_DEMO_TIMER, c, dm ? kDemoRespawnTime + kDt : 0.f);
    d.seti(CARL_CAR_CONTACT_IDX, c, -1);
    d.setf(CARL_CAR_CONTACT_COOLDOWN, c, 0.f);
    d.seti(CARL_CAR_BALL_HIT_TICK, c, -1);
    d.seti(CARL_CAR_BALL_CONTACT_TICK, c, -1);
    for (int f = CARL_CAR_CTRL_THROTTLE; f <= CARL_CAR_CTRL_SLIDE; f++) d.seti(f, c, 0);
    if (internal) {
        const float* v = internal + (size_t)src * kInternalFields;
        for (int f = CARL_CAR_ON_GROUND; f <= CARL_CAR_TIME_SINCE_BOOSTED; f++) d.seti(f, c, 0);
        d.seti(CARL_CAR_ON_GROUND, c, v[0] != 0.f);
        d.setf(CARL_CAR_AIR_TIME_SINCE_JUMP, c, v[1]);
        d.setf(CARL_CAR_HANDBRAKE, c, v[2]);
        d.seti(CARL_CAR_HAS_JUMPED, c, v[3] != 0.f);
        d.seti(CARL_CAR_IS_JUMPING, c, v[4] != 0.f);
        d.seti(CARL_CAR_LAST_JUMP, c, v[5] != 0.f);
        d.setf(CARL_CAR_JUMP_TIME, c, v[6]);
        d.seti(CARL_CAR_HAS_DOUBLE_JUMPED, c, v[7] != 0.f);
        d.seti(CARL_CAR_HAS_FLIPPED, c, v[8] != 0.f);
        d.seti(CARL_CAR_IS_FLIPPING, c, v[9] != 0.f);
        d.setf(CARL_CAR_FLIP_TIME, c, v[10]);
        d.seti(CARL_CAR_IS_AUTO_FLIPPING, c, v[11] != 0.f);
        d.setf(CARL_CAR_AUTO_FLIP_TIMER, c, v[12]);
        d.setf(CARL_CAR_AUTO_FLIP_SCALE, c, v[13]);
        d.setv(CARL_CAR_FLIP_TORQUE, c, V3{ v[14], v[15], v[16] });
        d.seti(CARL_CAR_IS_BOOSTING, c, v[17] != 0.f);
        d.setf(CARL_CAR_BOOSTING_TIME, c, v[18]);
        d.setf(CARL_CAR_BOOST, c, boost ? fmin_(kBoostMax, fmax_(0.f, boost[src])) : prevBoost);
    } else if (boost) {
        d.setf(CARL_CAR_BOOST, c, fmin_(kBoostMax, fmax_(0.f, boost[src])));
    }
    d.seti(CARL_CAR_CTRL_JUMP, c, d.ci(CARL_CAR_LAST_JUMP, c));
    d.setf(CARL_CAR_BRAKE_STAGE, c, 0.f);
    d.setf(CARL_CAR_STEER_STAGE, c, 0.f);
    d.setf(CARL_CAR_DRIVE_STAGE, c, 0.f);
    d.seti(CARL_CAR_MANIFOLD_COUNT, c, 0);
    for (int k = 0; k < kWheels; k++) {
        d.seti(CARL_CAR_WHEEL_CONTACT + k, c, 0);
        d.setf(CARL_CAR_LAT_FRICTION + k, c, 0.f);
        d.setf(CARL_CAR_LON_FRICTION + k, c, 0.f);
    }
}

// after a car restore: a demoed car has no wheel contacts and is airborne
DI void clearWheelContacts(const Dev& d, int c)
{
    for (int k = 0; k < kWheels; k++) {
        d.seti(CARL_CAR_WHEEL_SOURCE + k, c, kSrcNone);
        d.seti(CARL_CAR_WHEEL_CONTACT + k, c, 0);
    }
    d.seti(CARL_CAR_ON_GROUND, c, 0);
}

// suspension raycast against the restored scene; grounded = 3+ wheels
DI void storeRefreshedWheels(const Dev& d, int c, const Wheels& w)
{
    storeWheelOutputs(d, c, w);
    int n = 0;
    for (int k = 0; k < kWheels; k++) n += (w.src[k] != kSrcNone && w.dist[k] <= wheelRay(k)) ? 1 : 0;
    d.seti(CARL_CAR_ON_GROUND, c, n >= 3 ? 1 : 0);
}

}  // namespace carl
