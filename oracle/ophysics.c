/*
 * ophysics.c - the CARL physics tick, restated on the CPU.
 *
 * TEST INFRASTRUCTURE (see omath.h).  One call of ophys_tick runs the stages of
 * RLEnvironment::step (src/RLEnvironment.cu:166-211) over every car / sim in
 * the same stage order, so cross-car reads see the same values as the
 * reference's kernel sequence.  Per-stage citations are on each function.
 *
 * Ordering choices where the reference's result depends on thread timing:
 *   - car-triangle SAT hits are recorded in cell-list order (ascending
 *     triangle index) instead of atomicAdd order; at most 32 are kept;
 *   - the global tick counter is reset to 0 before every full reset.
 */
#include <stdlib.h>
#include <string.h>

#include "ointernal.h"

/* ------------------------------------------------------------------ tables */

/* The 120 kickoff permutations (src/RLConstants.cu:4-29): for each excluded
 * spawn e = 0..4 in turn, the lexicographic permutations of the other four. */
int ophys_kickoff_perm(int idx, int slot)
{
    const int excluded = idx / 24;
    int rest[4], n = 0;
    for (int i = 0; i < 5; i++) if (i != excluded) rest[n++] = i;
    int r = idx % 24;
    int fact[4] = { 6, 2, 1, 1 };
    int out[4];
    int used[4] = { 0, 0, 0, 0 };
    for (int p = 0; p < 4; p++) {
        int q = r / fact[p];
        r %= fact[p];
        for (int j = 0; j < 4; j++) {
            if (used[j]) continue;
            if (q == 0) { out[p] = rest[j]; used[j] = 1; break; }
            q--;
        }
    }
    return out[slot];
}

typedef struct { float x, y, z, yaw; } OSpawn;

static OSpawn kickoff_loc(int i)
{
    static const float xs[5] = { -2048.f, 2048.f, -256.f, 256.f, 0.f };
    static const float ys[5] = { -2560.f, -2560.f, -3840.f, -3840.f, -4608.f };
    const float yaw[5] = { K_PI_4 * 1, K_PI_4 * 3, K_PI_4 * 2, K_PI_4 * 2, K_PI_4 * 2 };
    OSpawn s = { xs[i], ys[i], K_CAR_REST_Z, yaw[i] };
    return s;
}

static OSpawn respawn_loc(int i)
{
    static const float xs[4] = { 2688.f, 2304.f, -2304.f, -2688.f };
    OSpawn s = { xs[i], -4608.f, K_CAR_REST_Z, K_PI_2 * 1 };
    return s;
}

/* include/Physics/BoostPads.cuh:21-56 */
static const float PAD_XYZ[N_PADS][3] = {
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

V3 ophys_pad_pos(int p) { return v3(PAD_XYZ[p][0], PAD_XYZ[p][1], PAD_XYZ[p][2]); }

/* --------------------------------------------------------------- integration */

/* include/Physics/Integration.cuh:6-39 */
Q4 ophys_integrate_quat(Q4 rot, V3 ang)
{
    const float dt = K_DT;
    const float maxMotion = K_ANG_MOTION_THRESH;
    const float angSpeedSq = vlensq(ang);
    float angSpeed = angSpeedSq > 1e-8f ? sqrtf(angSpeedSq) : 0.f;
    if (angSpeed * dt > maxMotion) angSpeed = maxMotion / dt;
    V3 axis;
    if (angSpeed < 0.001f) {
        const float dtSq = dt * dt;
        const float scale = 0.5f * dt - dtSq * dt * 0.020833333333f * angSpeed * angSpeed;
        axis = vscale(ang, scale);
    } else {
        axis = vscale(ang, o_sin(0.5f * angSpeed * dt) / angSpeed);
    }
    const Q4 delta = q4(axis.x, axis.y, axis.z, o_cos(0.5f * angSpeed * dt));
    const Q4 basis = qfromaxes(qworld(rot, V_X), qworld(rot, V_Y), qworld(rot, V_Z));
    return qnormalize(qcomp(delta, basis));
}

/* include/Physics/Integration.cuh:41-51 */
static void integrate_state(V3* pos, V3* cen, Q4* rot, V3 vel, V3 ang)
{
    *pos = vadd(*pos, vscale(vel, K_DT));
    *rot = ophys_integrate_quat(*rot, ang);
    *cen = vadd(*pos, qworld(*rot, K_CAR_OFFSETS));
}

/* ------------------------------------------------------------------ broadphase */

/* include/AABB.cuh:13-34 */
static V3 car_aabb_min(V3 cen, Q4 rot)
{
    const V3 rx = qworld(rot, V_X), ry = qworld(rot, V_Y), rz = qworld(rot, V_Z);
    const V3 half = vadd(vadd(vscale(vabs(rx), K_CAR_HALF.x), vscale(vabs(ry), K_CAR_HALF.y)),
                         vscale(vabs(rz), K_CAR_HALF.z));
    return vsub(cen, half);
}

/* include/Physics/CarArena/BroadPhase.cuh:10-28 */
void ophys_broadphase(OWorld* w, int ci)
{
    OCar* c = &w->cars[ci];
    V3 pos = c->pos, cen;
    Q4 rot = c->rot;
    integrate_state(&pos, &cen, &rot, c->vel, c->ang);
    const V3 swept = vmin(car_aabb_min(c->cen, c->rot), car_aabb_min(cen, rot));
    int cx, cy, cz;
    oarena_cell3(swept, &cx, &cy, &cz);
    c->cellIdx = oarena_flat(cx, cy, cz);
    c->numTris = w->arena->cellPrefix[c->cellIdx + 1] - w->arena->cellPrefix[c->cellIdx];
    c->hitCount = 0;
}

/* ------------------------------------------------------------------ raycast */

typedef struct { float dist; V3 normal; int source; } ORay;

static V3 ray_start(V3 cen, Q4 rot, int w) { return vadd(cen, qworld(rot, susp_connection(w))); }

/* include/Physics/SuspensionRaycast.cuh:25-44 */
static int ray_sphere(V3 start, V3 dir, V3 center, float radius, float maxDist, float* dist)
{
    const V3 off = vsub(start, center);
    const float b = vdot(off, dir);
    const float c = vlensq(off) - radius * radius;
    if (c < 0.f) return 0;
    const float disc = b * b - c;
    if (disc < 0.f) return 0;
    *dist = -b - sqrtf(disc);
    return *dist > 0.f && *dist <= maxDist;
}

/* include/Physics/SuspensionRaycast.cuh:46-94 */
static int ray_obb(V3 start, V3 dir, V3 center, Q4 rot, V3 half, float maxDist, float* dist, V3* normal)
{
    const V3 ls = qlocal(rot, vsub(start, center));
    const V3 ld = qlocal(rot, dir);
    float entry = 0.f, exitD = maxDist;
    int hitAxis = -1;
    for (int a = 0; a < 3; a++) {
        const float d = vget(ld, a), s = vget(ls, a), h = vget(half, a);
        if (fabsf(d) < 1e-8f) {
            if (fabsf(s) > h) return 0;
            continue;
        }
        const float inv = 1.f / d;
        const float t1 = (-h - s) * inv;
        const float t2 = (h - s) * inv;
        const float tNear = o_min(t1, t2);
        if (tNear > entry) { entry = tNear; hitAxis = a; }
        exitD = o_min(exitD, o_max(t1, t2));
        if (entry > exitD) return 0;
    }
    if (hitAxis < 0) return 0;
    *dist = entry;
    V3 ln = V_ZERO;
    vset(&ln, hitAxis, vget(ld, hitAxis) > 0.f ? -1.f : 1.f);
    *normal = qworld(rot, ln);
    return 1;
}

void ophys_init_empty_wheels(OCar* c, V3 up)
{
    for (int k = 0; k < N_WHEELS; k++) {
        c->rayDist[k] = susp_ray_len(k) + 1.f;
        c->rayNormal[k] = up;
        c->wheelSource[k] = SRC_NONE;
        c->wheelContact[k] = 0;
    }
}

/* include/Physics/SuspensionRaycast.cuh:98-301 */
void ophys_raycast(OWorld* w, int ci)
{
    OCar* c = &w->cars[ci];
    const OArena* A = w->arena;
    const V3 cen = c->cen;
    const Q4 rot = c->rot;
    const V3 up = qworld(rot, V_Z);
    const V3 dir = vneg(up);
    const int sim = ci / w->nCars;
    ORay best[N_WHEELS];
    for (int k = 0; k < N_WHEELS; k++) { best[k].dist = susp_ray_len(k) + 1.f; best[k].normal = up; best[k].source = SRC_NONE; }

    /* arena triangles of the broadphase cell (Moller-Trumbore) */
    const int start = A->cellPrefix[c->cellIdx];
    for (int i = 0; i < c->numTris; i++) {
        const int t = A->cellTris[start + i];
        const V3 p0 = A->verts[A->tris[3 * t]];
        const V3 e1 = vsub(A->verts[A->tris[3 * t + 1]], p0);
        const V3 e2 = vsub(A->verts[A->tris[3 * t + 2]], p0);
        const V3 pv = vcross(dir, e2);
        const float det = vdot(e1, pv);
        if (fabsf(det) < 1e-8f) continue;
        const float invDet = 1.f / det;
        for (int k = 0; k < N_WHEELS; k++) {
            const V3 tv = vsub(ray_start(cen, rot, k), p0);
            const float u = invDet * vdot(tv, pv);
            if (u < 0.f || u > 1.f) continue;
            const V3 qv = vcross(tv, e1);
            const float v = invDet * vdot(dir, qv);
            if (v < 0.f || u + v > 1.f) continue;
            const float hd = invDet * vdot(e2, qv);
            if (hd <= 0.f || hd >= best[k].dist) continue;
            best[k].dist = hd;
            best[k].source = SRC_ARENA;
            V3 fn = vcross(e1, e2);
            const float nl = vlensq(fn);
            if (nl > 1e-12f) {
                fn = vscale(fn, o_rsqrt(nl));
                if (vdot(fn, dir) > 0.f) fn = vneg(fn);
                best[k].normal = fn;
            }
        }
    }

    /* other cars of the simulation (slab OBB) */
    for (int o = 0; o < w->nCars; o++) {
        const int oi = sim * w->nCars + o;
        if (oi == ci) continue;
        if (w->cars[oi].demoed) continue;
        const V3 ocen = w->cars[oi].cen;
        const Q4 orot = w->cars[oi].rot;
        for (int k = 0; k < N_WHEELS; k++) {
            float d; V3 n;
            const int hit = ray_obb(ray_start(cen, rot, k), dir, ocen, orot, K_CAR_HALF, susp_ray_len(k), &d, &n);
            if (!hit || d >= best[k].dist) continue;
            best[k].dist = d; best[k].normal = n; best[k].source = SRC_CAR;
        }
    }

    /* ball */
    const V3 ball = w->sims[sim].pos;
    const float invR = 1.f / K_BALL_RADIUS;
    for (int k = 0; k < N_WHEELS; k++) {
        float d;
        const V3 rs = ray_start(cen, rot, k);
        const int hit = ray_sphere(rs, dir, ball, K_BALL_RADIUS, susp_ray_len(k), &d);
        if (!hit || d >= best[k].dist) continue;
        best[k].dist = d;
        best[k].normal = vscale(vsub(vadd(rs, vscale(dir, d)), ball), invR);
        best[k].source = SRC_BALL;
    }

    for (int k = 0; k < N_WHEELS; k++) {
        c->rayDist[k] = best[k].dist;
        c->rayNormal[k] = best[k].normal;
        c->wheelSource[k] = best[k].source;
        c->wheelContact[k] = best[k].source != SRC_NONE && best[k].dist <= susp_ray_len(k);
    }
}

/* ------------------------------------------------------------------ controls */

/* include/State/Controls.cuh:57-112 */
void ophys_controls_decode(int kind, const void* actions, int ci, OControls* out)
{
    if (kind == 0) {
        const int32_t* a = (const int32_t*)actions + 7 * ci;
#define AXIS_D(v) ((v) == 1 ? -1.f : ((v) == 2 ? 1.f : 0.f))
        const float h = AXIS_D(a[0]);
        out->throttle = AXIS_D(a[2]); out->steer = h; out->yaw = h;
        out->pitch = AXIS_D(a[1]); out->roll = AXIS_D(a[5]);
        out->jump = a[6] == 1; out->boost = a[4] == 1; out->slide = a[3] == 1;
#undef AXIS_D
    } else if (kind == 1) {
        const float* a = (const float*)actions + 7 * ci;
#define AXIS_C(v) ((v) < -1.f ? -1.f : ((v) > 1.f ? 1.f : (v)))
        const float h = AXIS_C(a[0]);
        out->throttle = AXIS_C(a[2]); out->steer = h; out->yaw = h;
        out->pitch = AXIS_C(a[1]); out->roll = AXIS_C(a[5]);
        out->jump = a[6] >= .5f; out->boost = a[4] >= .5f; out->slide = a[3] >= .5f;
#undef AXIS_C
    } else {
        const char* base = (const char*)actions + 32 * (size_t)ci;
        float f[5]; int32_t i3[3];
        memcpy(f, base, 20); memcpy(i3, base + 20, 12);
        out->throttle = f[0]; out->steer = f[1]; out->yaw = f[2]; out->pitch = f[3]; out->roll = f[4];
        out->jump = i3[0]; out->boost = i3[1]; out->slide = i3[2];
    }
}

typedef struct {
    OWorld* w;
    OCar* c;
    Q4 rot;
    V3 fwd, up;
    float fwdSpeed, absFwdSpeed;
    int wheelCount, onGround, jumpPressed;
} OCtx;

static float steer_angle_from_speed(float x)
{
    if (x <= 0.f) return 0.53356f;
    if (x <= 500.f) return 0.53356f + (0.31930f - 0.53356f) * (x / 500.f);
    if (x <= 1000.f) return 0.31930f + (0.18203f - 0.31930f) * ((x - 500.f) / 500.f);
    if (x <= 1500.f) return 0.18203f + (0.10570f - 0.18203f) * ((x - 1000.f) / 500.f);
    if (x <= 1750.f) return 0.10570f + (0.08507f - 0.10570f) * ((x - 1500.f) / 250.f);
    if (x <= 3000.f) return 0.08507f + (0.03454f - 0.08507f) * ((x - 1750.f) / 1250.f);
    return 0.03454f;
}

static float powerslide_steer_angle(float x)
{
    if (x <= 0.f) return 0.39235f;
    if (x <= 2500.f) return 0.39235f + (0.12610f - 0.39235f) * (x / 2500.f);
    return 0.12610f;
}

static float drive_torque_factor(float x)
{
    if (x <= 0.f) return 1.f;
    if (x >= 1410.f) return 0.f;
    if (x <= 1400.f) return 1.f - (x / 1400.f) * 0.9f;
    return 0.1f * (1.f - (x - 1400.f) / 10.f);
}

/* include/Physics/Controls/Drive.cuh:42-93 */
static void ground_drive(OCtx* x)
{
    OCar* c = x->c;
    const float throttle = (c->ctrl.boost && c->in.boost > 0.f) ? 1.f : c->ctrl.throttle;
    const int opposing = x->absFwdSpeed > K_STOPPING_VEL && ((throttle > 0.f) != (x->fwdSpeed > 0.f));
    float brake;
    if (x->wheelCount == 0 || c->ctrl.slide) brake = 0.f;
    else if (fabsf(throttle) >= K_THROTTLE_DEADZONE) brake = opposing ? 1.f : 0.f;
    else brake = x->absFwdSpeed < K_STOPPING_VEL ? 1.f : K_COASTING_BRAKE;
    float drive;
    if (x->wheelCount == 0) drive = 0.f;
    else if (fabsf(throttle) < K_THROTTLE_DEADZONE) drive = 0.f;
    else if (!c->ctrl.slide && opposing) drive = 0.f;
    else {
        float scale = drive_torque_factor(x->absFwdSpeed);
        if (x->wheelCount < 3) scale *= 0.25f;
        drive = throttle * K_THROTTLE_GROUND_ACCEL * scale;
    }
    c->brakePrev = c->brake; c->brake = brake;
    c->throttleVal = throttle;
    c->rawThrottle = c->ctrl.throttle;
    c->drivePrev = c->drive; c->drive = drive;
}

/* include/Physics/Controls/Drive.cuh:95-121 */
static void update_boost(OCtx* x)
{
    OInternal* s = &x->c->in;
    const OControls* k = &x->c->ctrl;
    int boosting;
    if (s->boost <= 0.f) boosting = 0;
    else if (!s->isBoosting) boosting = k->boost;
    else boosting = k->boost || s->boostingTime < K_BOOST_MIN_TIME;
    s->isBoosting = boosting;
    if (s->isBoosting) {
        s->boostingTime += K_DT;
        s->boost = o_max(s->boost - K_BOOST_PER_SECOND * K_DT, 0.f);
        const float accel = x->onGround ? K_BOOST_ACCEL_GROUND : K_BOOST_ACCEL_AIR;
        x->c->jumpImp = vadd(x->c->jumpImp, vscale(x->fwd, accel * K_DT));
        s->timeSinceBoosted = 0.f;
    } else {
        s->boostingTime = 0.f;
        s->timeSinceBoosted += K_DT;
    }
    s->boost = o_min(s->boost, K_BOOST_MAX);
}

/* include/Physics/Controls/Drive.cuh:123-146 */
static void update_steer(OCtx* x)
{
    OInternal* s = &x->c->in;
    const OControls* k = &x->c->ctrl;
    if (k->slide) s->handbrake += K_POWERSLIDE_RISE * K_DT;
    else s->handbrake -= K_POWERSLIDE_FALL * K_DT;
    s->handbrake = o_clamp(s->handbrake, 0.f, 1.f);
    x->c->handbrakeVal = s->handbrake;
    float angle = steer_angle_from_speed(x->absFwdSpeed);
    if (s->handbrake > 0.f) {
        const float slide = powerslide_steer_angle(x->absFwdSpeed);
        angle += (slide - angle) * s->handbrake;
    }
    x->c->steerPrev = x->c->steer;
    x->c->steer = angle * k->steer;
}

/* include/Physics/Controls/Aerial.cuh:244-275 */
static int apply_flip_torque(OCtx* x)
{
    OInternal* s = &x->c->in;
    const OControls* k = &x->c->ctrl;
    if (s->isFlipping) s->isFlipping = s->hasFlipped && s->flipTime < K_FLIP_TORQUE_TIME;
    if (!s->isFlipping) return 1;
    const V3 rel = s->flipTorque;
    if (vlensq(rel) <= 1e-12f) return 1;
    float pitchScale = 1.f;
    int useAir = 0;
    const int hasPitch = rel.y != 0.f && k->pitch != 0.f;
    const int matches = (rel.y > 0.f) == (k->pitch > 0.f);
    if (hasPitch && matches) {
        pitchScale = 1.f - o_min(fabsf(k->pitch), 1.f);
        useAir = 1;
    }
    const V3 relTorque = v3(rel.x * K_FLIP_TORQUE_X, rel.y * K_FLIP_TORQUE_Y * pitchScale, 0.f);
    const V3 world = qworld(x->rot, relTorque);
    x->c->angImp = vadd(x->c->angImp, vscale(world, K_DT));
    return useAir;
}

static V3 air_axis(const OCtx* x, int a)
{
    if (a == 0) return vneg(qworld(x->rot, V_Y));
    if (a == 1) return x->up;
    return vneg(x->fwd);
}

/* include/Physics/Controls/Aerial.cuh:277-326 */
static void apply_air_torque(OCtx* x)
{
    const OInternal* s = &x->c->in;
    const OControls* k = &x->c->ctrl;
    const int locked = s->isFlipping || (s->hasFlipped && s->flipTime < K_FLIP_TORQUE_TIME + K_FLIP_PITCHLOCK_EXTRA);
    const float pitchScale = locked ? 0.f : 1.f;
    const V3 input = v3(k->pitch, k->yaw, k->roll);
    const V3 controlScale = v3(pitchScale, 1.f, 1.f);
    const V3 dampInput = v3(k->pitch * pitchScale, k->yaw, 0.f);
    const V3 ang = x->c->ang;
    V3 torque = V_ZERO, damping = V_ZERO;
    const int hasInput = vlensq(input) > 0.f;
    for (int i = 0; i < 3; i++) {
        const V3 dir = air_axis(x, i);
        const float control = vget(input, i) * vget(controlScale, i);
        const float proj = vdot(dir, ang);
        const float damp = proj * K_AIR_DAMPING[i] * (1.f - fabsf(vget(dampInput, i)));
        if (hasInput) torque = vadd(torque, vscale(dir, control * K_AIR_TORQUE[i]));
        damping = vadd(damping, vscale(dir, damp));
    }
    x->c->angImp = vadd(x->c->angImp, vscale(vsub(torque, damping), K_TORQUE_SCALE * K_DT));
}

/* include/Physics/Controls/Aerial.cuh:328-342 */
static void update_air_control(OCtx* x, int allowAir)
{
    const int useAir = apply_flip_torque(x);
    if (useAir && allowAir && !x->c->in.isAutoFlipping) apply_air_torque(x);
    if (x->c->ctrl.throttle != 0.f)
        x->c->jumpImp = vadd(x->c->jumpImp, vscale(x->fwd, x->c->ctrl.throttle * K_THROTTLE_AIR_ACCEL * K_DT));
}

/* include/Physics/Controls/Aerial.cuh:15-73 */
static void update_jump(OCtx* x)
{
    OInternal* s = &x->c->in;
    const OControls* k = &x->c->ctrl;
    const int grace = s->hasJumped && s->jumpTime < K_JUMP_MIN_TIME + K_JUMP_RESET_PAD;
    if (x->onGround && !s->isJumping && !grace) { s->hasJumped = 0; s->jumpTime = 0.f; }
    if (s->isJumping) {
        s->isJumping = s->jumpTime < K_JUMP_MIN_TIME || (k->jump && s->jumpTime < K_JUMP_MAX_TIME);
    } else if (x->onGround && x->jumpPressed) {
        s->isJumping = 1;
        s->jumpTime = 0.f;
        x->c->jumpImp = vadd(x->c->jumpImp, vscale(x->up, K_JUMP_IMMEDIATE));
    }
    if (s->isJumping) {
        s->hasJumped = 1;
        float accel = K_JUMP_ACCEL;
        if (s->jumpTime < K_JUMP_MIN_TIME) accel *= 0.62f;
        x->c->jumpImp = vadd(x->c->jumpImp, vscale(x->up, accel * K_DT));
    }
    if (s->isJumping || s->hasJumped) s->jumpTime += K_DT;
}

/* include/Physics/Controls/Drive.cuh:134-178 */
static void update_autoflip(OCtx* x)
{
    OInternal* s = &x->c->in;
    if (x->jumpPressed && x->c->manCount != 0) {
        const V3 n = x->c->manNormal;
        if (n.z > K_AUTOFLIP_NORMZ) {
            const V3 right = qworld(x->rot, V_Y);
            const float roll = -o_atan2(right.z, x->up.z);
            const float absRoll = fabsf(roll);
            if (absRoll > K_AUTOFLIP_ROLL) {
                s->autoFlipTimer = K_AUTOFLIP_TIME * (absRoll / K_PI);
                s->autoFlipScale = roll > 0.f ? 1.f : -1.f;
                s->isAutoFlipping = 1;
                x->c->vel = vadd(x->c->vel, vscale(x->up, -K_AUTOFLIP_IMPULSE));
            }
        }
    }
    if (!s->isAutoFlipping) return;
    if (s->autoFlipTimer <= 0.f) { s->isAutoFlipping = 0; s->autoFlipTimer = 0.f; return; }
    const float torque = K_AUTOFLIP_TORQUE * s->autoFlipScale * K_DT;
    x->c->ang = vadd(x->c->ang, vscale(x->fwd, torque));
    s->autoFlipTimer -= K_DT;
}

/* include/Physics/Controls/Aerial.cuh:75-193 */
static void start_flip(OCtx* x, V3 dodge)
{
    OInternal* s = &x->c->in;
    s->flipTime = 0.f; s->hasFlipped = 1; s->isFlipping = 1;
    if (fabsf(dodge.x) < 0.1f && fabsf(dodge.y) < 0.1f) dodge = V_ZERO;
    else dodge = vscale(dodge, o_rsqrt(vlensq(dodge)));
    s->flipTorque = v3(-dodge.y, dodge.x, 0.f);

    /* scaledDodgeVel */
    V3 d = dodge;
    if (fabsf(d.x) < 0.1f) d.x = 0.f;
    if (fabsf(d.y) < 0.1f) d.y = 0.f;
    const float speedScale = o_clamp(x->absFwdSpeed / K_CAR_MAX_SPEED, 0.f, 1.f);
    int backward;
    if (x->absFwdSpeed < 100.f) backward = d.x < 0.f;
    else backward = (d.x >= 0.f) != (x->fwdSpeed >= 0.f);
    const float maxFwd = backward ? K_FLIP_BACK_SCALE : K_FLIP_FWD_SCALE;
    V3 lv = vscale(d, K_FLIP_INITIAL_VEL);
    lv.x *= (maxFwd - 1.f) * speedScale + 1.f;
    lv.y *= (K_FLIP_SIDE_SCALE - 1.f) * speedScale + 1.f;
    if (backward) lv.x *= K_FLIP_BACK_X;

    /* worldDodgeVel */
    const V3 flat = v3(x->fwd.x, x->fwd.y, 0.f);
    const float den = vlensq(flat);
    const V3 flatN = den > 1e-12f ? vscale(flat, o_rsqrt(den)) : V_X;
    const V3 right = v3(-flatN.y, flatN.x, 0.f);
    x->c->vel = vadd(x->c->vel, vadd(vscale(flatN, lv.x), vscale(right, lv.y)));
}

static void try_start_dodge(OCtx* x)
{
    OInternal* s = &x->c->in;
    const OControls* k = &x->c->ctrl;
    const int canDodge = !s->hasFlipped && !s->hasDoubleJumped && s->airTimeSinceJump < K_DOUBLEJUMP_MAX_DELAY;
    if (!x->jumpPressed || !canDodge) return;
    const V3 dodge = v3(-k->pitch, k->yaw + k->roll, 0.f);
    const float mag = fabsf(k->yaw) + fabsf(k->pitch) + fabsf(k->roll);
    if (mag >= K_DODGE_DEADZONE) { start_flip(x, dodge); return; }
    x->c->vel = vadd(x->c->vel, vscale(x->up, K_JUMP_IMMEDIATE));
    s->hasDoubleJumped = 1;
}

static void update_dodge(OCtx* x)
{
    OInternal* s = &x->c->in;
    if (x->onGround) {
        s->hasDoubleJumped = 0; s->hasFlipped = 0; s->isFlipping = 0;
        s->airTime = 0.f; s->airTimeSinceJump = 0.f; s->flipTime = 0.f;
    } else {
        s->airTime += K_DT;
        if (s->hasJumped && !s->isJumping) s->airTimeSinceJump += K_DT;
        else s->airTimeSinceJump = 0.f;
        try_start_dodge(x);
    }
    /* updateFlipMotion */
    if (!s->isFlipping) {
        if (s->hasFlipped) s->flipTime += K_DT;
        return;
    }
    s->flipTime += K_DT;
    if (s->flipTime > K_FLIP_TORQUE_TIME) return;
    V3 vel = x->c->vel;
    const int dampZ = s->flipTime >= K_FLIP_Z_DAMP_START && (vel.z < 0.f || s->flipTime < K_FLIP_Z_DAMP_END);
    if (!dampZ) return;
    vel.z *= 1.f - K_FLIP_Z_DAMP_120;
    x->c->vel = vel;
}

static void make_ctx(OWorld* w, OCar* c, OCtx* x)
{
    x->w = w; x->c = c;
    x->rot = c->rot;
    x->fwd = qworld(x->rot, V_X);
    x->up = qworld(x->rot, V_Z);
    x->fwdSpeed = vdot(c->vel, x->fwd);
    x->absFwdSpeed = fabsf(x->fwdSpeed);
    int n = 0;
    for (int k = 0; k < N_WHEELS; k++) if (c->rayDist[k] <= susp_ray_len(k)) n++;
    x->wheelCount = n;
    x->onGround = n >= 3;
    x->jumpPressed = c->ctrl.jump && !c->in.lastJump;
    c->in.lastJump = c->ctrl.jump;
    c->in.onGround = x->onGround;
}

/* include/Physics/Controls.cuh:7-35 */
static void process_controls(OWorld* w, OCar* c)
{
    if (c->demoed) { c->jumpImp = V_ZERO; c->angImp = V_ZERO; return; }
    OCtx x;
    make_ctx(w, c, &x);
    ground_drive(&x);
    update_boost(&x);
    update_steer(&x);
    if (x.wheelCount < 3) update_air_control(&x, x.wheelCount == 0);
    update_jump(&x);
    update_autoflip(&x);
    update_dodge(&x);
}

/* ------------------------------------------------------------ car-arena SAT */

typedef struct { V3 v0, v1, v2, e0, e1, e2, delta; } OTri;

static void tri_set(OTri* t, V3 a, V3 b, V3 c)
{
    t->v0 = a; t->v1 = b; t->v2 = c;
    t->e0 = vsub(b, a); t->e1 = vsub(c, b); t->e2 = vsub(a, c);
}

static V3 tri_center(const OTri* t) { return vdivs(vadd(vadd(t->v0, t->v1), t->v2), 3.f); }
static V3 tri_vert(const OTri* t, int i) { return i == 0 ? t->v0 : (i == 1 ? t->v1 : t->v2); }
static V3 tri_edge(const OTri* t, int i) { return i == 0 ? t->e0 : (i == 1 ? t->e1 : t->e2); }

typedef struct { int overlap, axisIdx; float minPen; V3 minAxis; } OSat;

/* include/Physics/CarArena/SAT.cuh:42-94 */
static void tri_axis(V3 ax, const OTri* t, int idx, int norm, OSat* r)
{
    if (!r->overlap) return;
    const float l = vlensq(ax);
    if (l < 1e-12f) return;
    if (norm) ax = vscale(ax, o_rsqrt(l));
    ax = vscale(ax, copysignf(1.f, vdot(ax, t->delta)));
    const float rr = vdot(vabs(ax), K_CAR_HALF);
    const float cMin = -rr, cMax = rr;
    const float d0 = vdot(t->v0, ax), d1 = vdot(t->v1, ax), d2 = vdot(t->v2, ax);
    const float tMin = o_min(o_min(d0, d1), d2);
    const float tMax = o_max(o_max(d0, d1), d2);
    if (cMax < tMin || tMax < cMin) { r->overlap = 0; return; }
    const float depth = o_min(cMax - tMin, tMax - cMin);
    if (depth < r->minPen) { r->minPen = depth; r->minAxis = ax; r->axisIdx = idx; }
}

static OSat tri_sat(const OTri* t)
{
    OSat r = { 1, 0, K_FLT_MAX, { 0.f, 0.f, 0.f } };
    tri_axis(vcross(t->e0, t->e1), t, 0, 1, &r);
    if (!r.overlap) return r;
    tri_axis(V_X, t, 1, 0, &r);
    tri_axis(V_Y, t, 2, 0, &r);
    tri_axis(V_Z, t, 3, 0, &r);
    for (int a = 0; a < 3; a++)
        for (int e = 0; e < 3; e++)
            tri_axis(vcross(tri_edge(t, e), v_axis(a)), t, 4 + 3 * a + e, 1, &r);
    return r;
}

/* include/Physics/CarArena/SAT.cuh:123-161, in cell-list order */
static void car_arena_sat(OWorld* w, int ci)
{
    OCar* c = &w->cars[ci];
    const OArena* A = w->arena;
    const int start = A->cellPrefix[c->cellIdx];
    c->hitCount = 0;
    for (int i = 0; i < c->numTris; i++) {
        const int t = A->cellTris[start + i];
        const V3 a = A->verts[A->tris[3 * t]], b = A->verts[A->tris[3 * t + 1]], cc = A->verts[A->tris[3 * t + 2]];
        const int horiz = a.z == b.z && a.z == cc.z && (a.z == 0.f || a.z == 2048.f);
        const int wall = a.x == b.x && a.x == cc.x && fabsf(a.x) == 4096.f;
        if (horiz || wall) continue;
        OTri tr;
        tri_set(&tr, qlocal(c->rot, vsub(a, c->cen)), qlocal(c->rot, vsub(b, c->cen)), qlocal(c->rot, vsub(cc, c->cen)));
        tr.delta = vneg(tri_center(&tr));
        const OSat s = tri_sat(&tr);
        if (!s.overlap) continue;
        const int slot = c->hitCount++;
        if (slot >= MAX_TRI_PAIRS) continue;
        OHit* h = &c->hits[slot];
        h->v0 = tr.v0; h->v1 = tr.v1; h->v2 = tr.v2; h->tri = t;
        h->axisIdx = s.axisIdx; h->minAxis = s.minAxis; h->minPen = s.minPen;
    }
}

/* ----------------------------------------------------------- car-arena clip */

typedef struct { OTri t; V3 faceNormal; V3 angles; } OTriClip;

static void load_tri_clip(const OWorld* w, const OHit* h, OTriClip* tc)
{
    tri_set(&tc->t, h->v0, h->v1, h->v2);
    tc->faceNormal = vnorm(vcross(tc->t.e0, vsub(tc->t.v2, tc->t.v0)));
    tc->angles = w->arena->angs[h->tri];
}

/* include/Physics/Collision/Clip.cuh:5-35; the output is capped at the 8-vertex
 * buffer size (exceeded only through rounding on near-degenerate polygons) */
#define MAX_POLYGON 8
static int clip_plane(const V3* in, int n, V3* out, V3 normal, float dist)
{
    if (n == 0) return 0;
    int o = 0;
    for (int i = 0; i < n; i++) {
        const V3 cur = in[i], nxt = in[(i + 1) % n];
        const float cd = vdot(normal, cur) - dist;
        const float nd = vdot(normal, nxt) - dist;
        const int ci = cd <= 0.f, ni = nd <= 0.f;
        if (ci && o < MAX_POLYGON) out[o++] = cur;
        if (ci != ni && o < MAX_POLYGON) {
            const float t = cd / (cd - nd);
            out[o++] = vadd(cur, vscale(vsub(nxt, cur), t));
        }
    }
    return o;
}

/* include/Physics/CarArena/Clip.cuh:163-218 */
static OContact edge_edge_contact(const OTriClip* tc, float minPen, int axisIdx, V3 sep)
{
    const int carAxis = (axisIdx - 4) / 3;
    const int triEdge = (axisIdx - 4) % 3;
    const V3 triCenter = tri_center(&tc->t);
    if (vdot(sep, triCenter) > 0.f) sep = vneg(sep);
    V3 carPoint = vmul(vsign(vneg(sep)), K_CAR_HALF);
    vset(&carPoint, carAxis, 0.f);
    const V3 carAx = v_axis(carAxis);
    const V3 triPoint = tri_vert(&tc->t, triEdge);
    const V3 edge = tri_edge(&tc->t, triEdge);
    const float triLen = vlen(edge);
    const V3 triAx = vdivs(edge, triLen);
    const V3 carToTri = vsub(triPoint, carPoint);
    const float axisDot = vdot(carAx, triAx);
    const float denom = 1.f - axisDot * axisDot;
    V3 onTri = triPoint;
    if (denom > 1e-6f) {
        const float carProj = vdot(carToTri, carAx);
        const float triProj = vdot(carToTri, triAx);
        const float un = (axisDot * carProj - triProj) / denom;
        const float tp = o_clamp(un, 0.f, triLen);
        onTri = vadd(triPoint, vscale(triAx, tp));
    }
    const float cpp = vdot(carAx, vsub(onTri, carPoint));
    const float half = vget(K_CAR_HALF, carAxis);
    const float cp = o_clamp(cpp, -half, half);
    const V3 onCar = vadd(carPoint, vscale(carAx, cp));
    const V3 sepv = vsub(onTri, onCar);
    const float sq = vlensq(sepv);
    OContact r;
    r.carPos = onCar; r.arenaPos = onTri; r.depth = minPen;
    if (sq > 1e-8f) {
        V3 n = vscale(sepv, o_rsqrt(sq));
        if (vdot(n, triCenter) > 0.f) n = vneg(n);
        r.normal = n;
    } else {
        r.normal = sep;
    }
    return r;
}

/* Contacts of one SAT-overlapping triangle (box-local vertices): the
 * edge-edge contact for an edge axis, else the triangle clipped to the
 * witness face's side planes (include/Physics/CarArena/Clip.cuh:244-377). */
static int clip_pair(const OTriClip* tc, int axisIdx, float minPen, V3 sep, OContact* out)
{
    if (axisIdx >= 4) {
        out[0] = edge_edge_contact(tc, minPen, axisIdx, sep);
        return 1;
    }
    V3 bufA[MAX_PAIR_CONTACTS], bufB[MAX_PAIR_CONTACTS];
    V3* in = bufA; V3* o = bufB;
    const int faceAxis = vargmax(vabs(sep));
    int cnt = 3;
    in[0] = tc->t.v0; in[1] = tc->t.v1; in[2] = tc->t.v2;
    for (int a = 0; a < 3 && cnt > 0; a++) {
        if (a == faceAxis) continue;
        for (int sg = 1; sg >= -1 && cnt > 0; sg -= 2) {
            cnt = clip_plane(in, cnt, o, vscale(v_axis(a), (float)sg), vget(K_CAR_HALF, a));
            V3* sw = in; in = o; o = sw;
        }
    }
    /* writeFaceContacts */
    const V3 faceNormal = vscale(v_axis(faceAxis), -copysignf(1.f, vget(sep, faceAxis)));
    const float faceDist = vget(K_CAR_HALF, faceAxis);
    const float minDepth = -(minPen + K_CONTACT_BREAK);
    int k = 0;
    for (int i = 0; i < cnt; i++) {
        float depth = vdot(faceNormal, in[i]) - faceDist;
        depth = o_max(depth, minDepth);
        if (depth > K_CONTACT_BREAK) continue;
        OContact* ct = &out[k++];
        ct->carPos = vadd(in[i], vscale(sep, depth));
        ct->arenaPos = in[i];
        ct->normal = sep;
        ct->depth = -depth;
    }
    return k;
}

static void car_arena_clip(OWorld* w, int ci)
{
    OCar* c = &w->cars[ci];
    const int n = c->hitCount < MAX_TRI_PAIRS ? c->hitCount : MAX_TRI_PAIRS;
    for (int p = 0; p < n; p++) {
        const OHit* h = &c->hits[p];
        OTriClip tc;
        load_tri_clip(w, h, &tc);
        c->conCount[p] = clip_pair(&tc, h->axisIdx, h->minPen, h->minAxis, c->contacts[p]);
    }
}

/* ------------------------------------------------------------------ manifold */

#define MAN_BREAK_SQ (K_CONTACT_BREAK * K_CONTACT_BREAK)

static int man_replacement(const OManPoint* pts, const OManPoint* cand)
{
    const V3 p0 = pts[0].carPos, p1 = pts[1].carPos, p2 = pts[2].carPos, p3 = pts[3].carPos;
    int deepest = -1;
    float deepestPen = -cand->dist;
    for (int i = 0; i < MAX_MANIFOLD; i++) {
        const float pen = -pts[i].dist;
        if (pen > deepestPen) { deepest = i; deepestPen = pen; }
    }
    float area[4] = { 0.f, 0.f, 0.f, 0.f };
    if (deepest != 0) area[0] = vlensq(vcross(vsub(cand->carPos, p1), vsub(p3, p2)));
    if (deepest != 1) area[1] = vlensq(vcross(vsub(cand->carPos, p0), vsub(p3, p2)));
    if (deepest != 2) area[2] = vlensq(vcross(vsub(cand->carPos, p0), vsub(p3, p1)));
    if (deepest != 3) area[3] = vlensq(vcross(vsub(cand->carPos, p0), vsub(p2, p1)));
    int best = 0;
    for (int i = 1; i < MAX_MANIFOLD; i++) if (area[i] > area[best]) best = i;
    return best;
}

static void man_add(OManPoint* pts, int* count, const OManPoint* p)
{
    int idx = *count;
    if (idx == MAX_MANIFOLD) idx = man_replacement(pts, p);
    else (*count)++;
    pts[idx] = *p;
}

static int man_nearby(const OManPoint* pts, int count, V3 carPos)
{
    for (int i = 0; i < count; i++)
        if (vlensq(vsub(pts[i].carPos, carPos)) < MAN_BREAK_SQ) return 1;
    return 0;
}

/* include/Physics/CarArena/Clip.cuh:53-161 */
static int clamp_normal(V3 edgeAxis, V3 triNormal, V3 contactNormal, float edgeAngle, V3* out)
{
    V3 ec = vcross(edgeAxis, triNormal);
    const float cl = vlensq(ec);
    if (cl <= 1e-12f) return 0;
    ec = vscale(ec, o_rsqrt(cl));
    const float tp = vdot(contactNormal, ec);
    const float np = vdot(contactNormal, triNormal);
    const float cur = o_atan2(tp, np);
    const int outside = edgeAngle < 0.f ? cur < edgeAngle : cur > edgeAngle;
    if (!outside) return 0;
    *out = o_rotate_axis(contactNormal, edgeAxis, edgeAngle - cur);
    return 1;
}

static void adjust_internal_edge(const OTriClip* tc, OContact* ct)
{
    if (vgte(tc->angles, K_BOUNDARY_EDGE_ANGLE)) return;
    int bestEdge = -1;
    float bestSq = K_FLT_MAX;
    for (int e = 0; e < 3; e++) {
        if (fabsf(vget(tc->angles, e)) >= K_BOUNDARY_EDGE_ANGLE) continue;
        const V3 s = tri_vert(&tc->t, e), en = tri_vert(&tc->t, (e + 1) % 3);
        const V3 seg = vsub(en, s);
        const float proj = vdot(vsub(ct->arenaPos, s), seg) / vlensq(seg);
        const V3 nearest = vadd(s, vscale(seg, o_clamp(proj, 0.f, 1.f)));
        const float sq = vlensq(vsub(ct->arenaPos, nearest));
        if (sq < bestSq) { bestSq = sq; bestEdge = e; }
    }
    if (bestEdge < 0 || bestSq >= 5.f * 5.f) return;
    const V3 localN = vnorm(ct->normal);
    const float angle = vget(tc->angles, bestEdge);
    if (angle == 0.f) {
        if (vdot(tc->faceNormal, localN) >= 0.f) {
            ct->normal = tc->faceNormal;
            ct->arenaPos = vadd(ct->carPos, vscale(tc->faceNormal, ct->depth));
        }
        return;
    }
    const float side = angle > 0.f ? 1.f : -1.f;
    const V3 edgeAxis = vnorm(tri_edge(&tc->t, bestEdge));
    const V3 nA = vscale(tc->faceNormal, side);
    const V3 nB = vscale(o_rotate_axis(tc->faceNormal, edgeAxis, angle), side);
    if (vdot(localN, nA) < 0.f && vdot(localN, nB) < 0.f) {
        if (vdot(tc->faceNormal, localN) >= 0.f) {
            ct->normal = tc->faceNormal;
            ct->arenaPos = vadd(ct->carPos, vscale(tc->faceNormal, ct->depth));
        }
        return;
    }
    V3 cl;
    if (clamp_normal(edgeAxis, nA, localN, angle, &cl) && vdot(cl, tc->faceNormal) > 0.f) {
        ct->normal = vnorm(cl);
        ct->arenaPos = vadd(ct->carPos, vscale(ct->normal, ct->depth));
    }
}

/* include/Physics/CarArena/Manifold.cuh:266-310 */
static int build_manifold(OWorld* w, int ci, OManPoint* pts)
{
    OCar* c = &w->cars[ci];
    const V3 cen = c->cen;
    const Q4 rot = c->rot;
    int count = 0;
    static const float offsets[4] = { 0.f, -2044.f, -4096.f, -4096.f };
    static const float normals[4][3] = { { 0.f, 0.f, 1.f }, { 0.f, 0.f, -1.f }, { 1.f, 0.f, 0.f }, { -1.f, 0.f, 0.f } };
    for (int p = 0; p < 4; p++) {
        const V3 n = v3(normals[p][0], normals[p][1], normals[p][2]);
        const V3 d = qlocal(rot, vneg(n));
        const V3 carPos = v3(d.x >= 0 ? K_CAR_HALF.x : -K_CAR_HALF.x,
                             d.y >= 0 ? K_CAR_HALF.y : -K_CAR_HALF.y,
                             d.z >= 0 ? K_CAR_HALF.z : -K_CAR_HALF.z);
        const V3 worldCar = vadd(cen, qworld(rot, carPos));
        const float dist = vdot(n, worldCar) - offsets[p];
        if (dist < K_CONTACT_BREAK && !man_nearby(pts, count, carPos)) {
            OManPoint mp;
            memset(&mp, 0, sizeof mp);
            mp.carPos = carPos; mp.worldPos = vsub(worldCar, vscale(n, dist)); mp.worldNormal = n;
            mp.dist = dist; mp.friction = K_WORLD_FRICTION; mp.restitution = K_WORLD_RESTITUTION;
            man_add(pts, &count, &mp);
        }
    }

    /* insertBestContact: the deepest clip contact not near an existing point */
    const int pairs = c->hitCount < MAX_TRI_PAIRS ? c->hitCount : MAX_TRI_PAIRS;
    int bestPair = -1;
    OContact best;
    memset(&best, 0, sizeof best);
    float bestDist = K_FLT_MAX;
    for (int p = 0; p < pairs; p++) {
        for (int k = 0; k < c->conCount[p]; k++) {
            const OContact* ct = &c->contacts[p][k];
            if (man_nearby(pts, count, ct->carPos)) continue;
            const float dist = -ct->depth;
            if (dist < bestDist) { bestDist = dist; best = *ct; bestPair = p; }
        }
    }
    if (bestPair >= 0) {
        OTriClip tc;
        load_tri_clip(w, &c->hits[bestPair], &tc);
        adjust_internal_edge(&tc, &best);
        OManPoint mp;
        memset(&mp, 0, sizeof mp);
        mp.carPos = best.carPos;
        mp.worldPos = vadd(cen, qworld(rot, best.arenaPos));
        mp.worldNormal = qworld(rot, best.normal);
        mp.dist = -best.depth;
        mp.friction = K_WORLD_FRICTION; mp.restitution = K_WORLD_RESTITUTION;
        man_add(pts, &count, &mp);
    }
    return count;
}

/* ---------------------------------------------------------------- solver body */

typedef struct {
    V3 pos, vel, ang, cen;
    Q4 rot;
    V3 extVel, extAng, deltaVel, deltaAng, pushVel, turnVel;
} OBody;

static OBody load_body(const OCar* c)
{
    OBody b;
    memset(&b, 0, sizeof b);
    b.pos = c->pos; b.vel = c->vel; b.ang = c->ang; b.cen = c->cen; b.rot = c->rot;
    b.extVel = vscale(K_GRAVITY, K_DT);
    return b;
}

static void store_body(OCar* c, const OBody* b)
{
    c->pos = b->pos; c->vel = b->vel; c->ang = b->ang; c->cen = b->cen; c->rot = b->rot;
}

static V3 inv_inertia_world(Q4 rot, V3 v) { return qworld(rot, vmul(qlocal(rot, v), K_CAR_INV_INERTIA)); }

/* include/Physics/CarArena/SolverBody.cuh:65-78 */
static void clamp_body(OBody* b)
{
    const float vs = vlensq(b->vel);
    if (vs > K_CAR_MAX_SPEED * K_CAR_MAX_SPEED) b->vel = vscale(b->vel, K_CAR_MAX_SPEED * o_rsqrt(vs));
    const float as = vlensq(b->ang);
    if (as > K_CAR_MAX_ANG * K_CAR_MAX_ANG) b->ang = vscale(b->ang, K_CAR_MAX_ANG * o_rsqrt(as));
}

/* include/Physics/Collision/Solver.cuh:5-60 */
static V3 fallback_tangent(V3 n)
{
    if (fabsf(n.z) > K_SQRT_1_2) {
        const float l = n.y * n.y + n.z * n.z;
        const float inv = o_rsqrt(l);
        return v3(0.f, -n.z * inv, n.y * inv);
    }
    const float l = n.x * n.x + n.y * n.y;
    const float inv = o_rsqrt(l);
    return v3(-n.y * inv, n.x * inv, 0.f);
}

static float solve_impulse(float rhs, float cfm, float jacInv, float relVel, float lower, float upper, float* applied)
{
    const float prev = *applied;
    const float delta = rhs - *applied * cfm - relVel * jacInv;
    *applied = o_clamp(prev + delta, lower, upper);
    return *applied - prev;
}

static float solve_lower(float rhs, float cfm, float jacInv, float relVel, float lower, float* applied)
{
    const float prev = *applied;
    const float delta = rhs - *applied * cfm - relVel * jacInv;
    *applied = o_max(prev + delta, lower);
    return *applied - prev;
}

/* ---------------------------------------------------------------- suspension */

static float non_sticky_friction(float z)
{
    if (z <= 0.f) return 0.1f;
    if (z >= 1.f) return 1.f;
    if (z < 0.7075f) return 0.1f + (z / 0.7075f) * 0.4f;
    return 0.5f + ((z - 0.7075f) / (1.f - 0.7075f)) * 0.5f;
}

typedef struct {
    V3 cenOffset, forward, right, up, vel, ang, angCrossUp;
    float brakeTorque, pushbackDt;
} OFrame;

/* include/Physics/CarSuspension.cuh:62-232 */
static void susp_wheel(const OBody* b, OCar* c, const OFrame* f, int w,
                       V3* directVel, V3* directAng, V3* deltaVel, V3* contactNorm, int* hasContact)
{
    *directVel = V_ZERO; *directAng = V_ZERO; *deltaVel = V_ZERO; *contactNorm = V_ZERO; *hasContact = 0;
    const float dist = c->rayDist[w];
    if (dist > susp_ray_len(w)) return;
    const float radius = susp_radius(w);
    const float rest = susp_rest(w);
    const float suspLen = o_min(o_max(dist - radius, rest - K_MAX_SUSP_TRAVEL), rest + K_MAX_SUSP_TRAVEL);
    const V3 normal = c->rayNormal[w];
    const V3 hardRel = vadd(f->cenOffset, qworld(b->rot, susp_connection(w)));
    const V3 fullRel = vsub(hardRel, vscale(f->up, dist));
    const V3 pointVel = vadd(f->vel, vcross(f->ang, fullRel));
    const float projVel = vdot(normal, pointVel);
    const float denom = vdot(normal, f->up);
    const float clipped = denom > 0.1f ? 1.f / denom : 10.f;
    const float relVel = projVel * clipped;
    const float damping = relVel < 0.f ? K_SUSP_DAMP_COMP : K_SUSP_DAMP_RELAX;
    float force = ((rest - suspLen) * K_SUSP_STIFFNESS - damping * projVel) * clipped * susp_scale(w);
    if (force <= 0.f) force = 0.f;
    float impulse = 0.f;
    if (force != 0.f) {
        impulse = force * K_DT;
        const float thr = rest + radius - K_SUSP_SUBTRACTION;
        if (dist < thr) {
            const float pen = thr - dist;
            const V3 ta = vcross(fullRel, normal);
            const V3 iit = inv_inertia_world(b->rot, ta);
            const float jac = K_CAR_INV_MASS + vdot(iit, ta);
            const float jacInv = 1.f / o_max(jac, 1e-8f);
            const float posErr = K_SUSP_PUSHBACK_ERP * pen / f->pushbackDt;
            const float velErr = -projVel;
            float push = (posErr + velErr) * jacInv;
            if (push < 0.f) push = 0.f;
            impulse += push * 0.25f;
        }
    }
    *deltaVel = vscale(normal, impulse * K_CAR_INV_MASS);
    *directAng = vscale(inv_inertia_world(b->rot, vcross(fullRel, normal)), impulse);

    V3 axle = f->right;
    if (w < 2) {
        const float steer = c->steerPrev;
        if (fabsf(steer) > 1e-6f) {
            float sn, cs;
            o_sincos(steer, &sn, &cs);
            axle = vadd(vscale(f->right, cs), vscale(vcross(f->up, f->right), sn));
        }
    }
    V3 axleDir = vsub(axle, vscale(normal, vdot(axle, normal)));
    const float axleSq = vlensq(axleDir);
    *contactNorm = normal;
    *hasContact = 1;
    if (axleSq <= 1e-10f) return;
    axleDir = vscale(axleDir, o_rsqrt(axleSq));
    const V3 latRel = vsub(fullRel, vscale(f->up, vdot(f->up, fullRel)));
    const V3 hardVel = vadd(pointVel, vscale(f->angCrossUp, dist));
    const V3 curveLong = vcross(axle, normal);
    const V3 fwdDir = vcross(normal, axleDir);
    float curveIn = 0.f;
    const float baseFric = fabsf(vdot(hardVel, axle));
    if (baseFric > 5.f) curveIn = baseFric / (fabsf(vdot(hardVel, curveLong)) + baseFric);
    const float hb = c->handbrakeVal;
    float latBase = 1.f - 0.8f * o_clamp(curveIn, 0.f, 1.f);
    float lonBase = 1.f;
    if (hb > 0.f) {
        latBase *= (0.1f - 1.f) * hb + 1.f;
        lonBase *= ((0.5f + 0.4f * o_clamp(curveIn, 0.f, 1.f)) - 1.f) * hb + 1.f;
    }
    const float nonSticky = non_sticky_friction(normal.z);
    const int sticky = c->throttleVal != 0.f;
    const float fs = sticky ? 1.f : nonSticky;
    const float latF = latBase * fs, lonF = lonBase * fs;
    const float latUsed = c->latF[w], lonUsed = c->lonF[w];
    c->latF[w] = latF; c->lonF[w] = lonF;
    const V3 ta = vcross(fullRel, axleDir);
    const V3 angLat = inv_inertia_world(b->rot, ta);
    const float jac = K_CAR_INV_MASS + vdot(axleDir, vcross(angLat, fullRel));
    const float latJacInv = 1.f / o_max(jac, 1e-8f);
    const float latVel = vdot(axleDir, pointVel);
    const float sideImp = -0.2f * latVel * latJacInv;
    const float lonVel = vdot(fwdDir, pointVel);
    const float drive = c->drivePrev;
    const float rolling = drive != 0.f ? -0.75f * drive
                                       : o_clamp(-lonVel * 113.73963f, -f->brakeTorque, f->brakeTorque);
    V3 wheelImp = vadd(vscale(axleDir, sideImp * latUsed), vscale(fwdDir, rolling * lonUsed));
    wheelImp = vscale(wheelImp, (K_CAR_MASS / 3.f) * K_DT);
    *directVel = vscale(wheelImp, K_CAR_INV_MASS);
    *directAng = vadd(*directAng, inv_inertia_world(b->rot, vcross(latRel, wheelImp)));
}

/* include/Physics/CarSuspension.cuh:234-339 */
static void apply_suspension(OBody* b, OCar* c, int tickCount)
{
    const float brakeTorque = c->brakePrev * (K_CAR_MASS * (14.25f + 1.f / 3.f));
    const V3 up = qworld(b->rot, V_Z);
    OFrame f;
    f.cenOffset = vsub(b->cen, b->pos);
    f.forward = qworld(b->rot, V_X);
    f.right = qworld(b->rot, V_Y);
    f.up = up;
    f.vel = b->vel;
    f.ang = b->ang;
    f.angCrossUp = vcross(b->ang, up);
    f.brakeTorque = brakeTorque;
    f.pushbackDt = tickCount <= 1 ? K_SUSP_PUSHBACK_DT_FIRST : K_DT;
    V3 normalSum = V_ZERO;
    int count = 0;
    for (int w = 0; w < N_WHEELS; w++) {
        V3 dv, da, dd, cn; int hc;
        susp_wheel(b, c, &f, w, &dv, &da, &dd, &cn, &hc);
        b->vel = vadd(b->vel, dv);
        b->ang = vadd(b->ang, da);
        b->deltaVel = vadd(b->deltaVel, dd);
        normalSum = vadd(normalSum, cn);
        count += hc;
    }

    /* applySuspAggregate, reading the previous tick's arena manifold */
    const float throttle = c->throttleVal;
    const int hasRaw = c->rawThrottle != 0.f;
    const int hasWorld = c->manCount != 0;
    V3 upDir;
    int autoroll = 0, skip = 0;
    if (count > 0) {
        upDir = vscale(normalSum, o_rsqrt(vlensq(normalSum) + 1e-16f));
        const float fwdSpeed = fabsf(vdot(f.vel, f.forward));
        const int fullStick = throttle != 0.f || fwdSpeed > K_STOPPING_VEL;
        float sticky = 0.5f;
        if (fullStick) sticky += 1.f - fabsf(upDir.z);
        b->extVel = vadd(b->extVel, vscale(upDir, sticky * K_GRAVITY.z * K_DT));
        autoroll = hasRaw && (count < N_WHEELS || hasWorld);
    } else if (hasWorld) {
        upDir = c->manNormal;
        autoroll = hasRaw;
    } else {
        skip = 1;
        upDir = V_ZERO;
    }
    if (!skip && autoroll) {
        const V3 down = vneg(upDir);
        const V3 crossRight = vcross(upDir, f.forward);
        const V3 crossFwd = vcross(down, crossRight);
        const float rtf = 1.f - o_clamp(vdot(f.right, crossRight), 0.f, 1.f);
        const float ftf = 1.f - o_clamp(vdot(f.forward, crossFwd), 0.f, 1.f);
        const V3 rightDir = vscale(f.forward, vdot(f.right, upDir) >= 0.f ? -1.f : 1.f);
        const V3 fwdDir = vscale(f.right, vdot(f.forward, upDir) >= 0.f ? 1.f : -1.f);
        b->deltaVel = vadd(b->deltaVel, vscale(down, K_AUTOROLL_FORCE * K_DT));
        b->deltaAng = vadd(b->deltaAng, vscale(vadd(vscale(fwdDir, ftf), vscale(rightDir, rtf)), K_AUTOROLL_TORQUE * K_DT));
    }

    b->extVel = vadd(b->extVel, c->jumpImp);
    c->jumpImp = V_ZERO;
    b->extAng = vadd(b->extAng, c->angImp);
    c->angImp = V_ZERO;
}

/* ------------------------------------------------------ car-arena solver rows */

typedef struct {
    V3 axis, relCross, angular;
    float jacInv, rhs, rhsPen, cfm, lower, upper, applied, appliedPush;
} ORow;

static ORow axis_row(const OBody* b, V3 axis, V3 relPos)
{
    ORow r;
    memset(&r, 0, sizeof r);
    r.axis = axis;
    r.relCross = vcross(relPos, axis);
    r.angular = inv_inertia_world(b->rot, r.relCross);
    const V3 lin = vcross(r.angular, relPos);
    const float denom = K_CAR_INV_MASS + vdot(axis, lin);
    r.jacInv = 1.f / o_max(denom, 1e-8f);
    r.upper = 1e10f;
    return r;
}

static float row_vel(const ORow* r, V3 lin, V3 ang) { return vdot(r->axis, lin) + vdot(r->relCross, ang); }

static void row_apply(OBody* b, const ORow* r, float imp)
{
    b->deltaVel = vadd(b->deltaVel, vscale(r->axis, K_CAR_INV_MASS * imp));
    b->deltaAng = vadd(b->deltaAng, vscale(r->angular, imp));
}

/* include/Physics/CarArena/Solve.cuh:206-264 */
static void solve_manifold(OBody* b, OManPoint* pts, int count)
{
    ORow nrm[MAX_MANIFOLD], fr[MAX_MANIFOLD];
    float fc[MAX_MANIFOLD];
    const V3 cenOffset = vsub(b->cen, b->pos);
    const V3 totalVel = vadd(b->vel, b->extVel);
    const V3 totalAng = vadd(b->ang, b->extAng);
    for (int i = 0; i < count; i++) {
        const OManPoint* p = &pts[i];
        const V3 relPos = vadd(cenOffset, qworld(b->rot, p->carPos));
        /* normal row */
        ORow n = axis_row(b, p->worldNormal, relPos);
        const float relVelNoExt = row_vel(&n, b->vel, b->ang);
        const float relVel = row_vel(&n, totalVel, totalAng);
        const float rest = fabsf(relVelNoExt) < K_RESTITUTION_VEL_THRESH ? 0.f : p->restitution * -relVelNoExt;
        const float pen = p->dist + K_LINEAR_SLOP;
        const float invDt = 1.f / K_DT;
        float posErr = 0.f;
        const float velErr = rest - relVel;
        if (pen <= 0.f) posErr = -pen * K_CONTACT_ERP * invDt;
        const float posImp = posErr * n.jacInv;
        const float velImp = velErr * n.jacInv;
        if (pen > K_SPLIT_PEN_THRESH) n.rhs = posImp + velImp;
        else { n.rhs = velImp; n.rhsPen = posImp; }
        n.applied = p->impulse * K_WARMSTART;
        /* friction row */
        const V3 cv = vadd(totalVel, vcross(totalAng, relPos));
        const float nv = vdot(p->worldNormal, cv);
        V3 tan = vsub(cv, vscale(p->worldNormal, nv));
        const float tl = vlensq(tan);
        tan = tl > 1e-8f ? vscale(tan, o_rsqrt(tl)) : fallback_tangent(p->worldNormal);
        ORow t = axis_row(b, tan, relPos);
        const float tv = row_vel(&t, totalVel, b->ang);
        t.rhs = -tv * t.jacInv;
        t.upper = 0.f;
        t.applied = 0.f;
        nrm[i] = n; fr[i] = t; fc[i] = p->friction;
        row_apply(b, &nrm[i], nrm[i].applied);   /* warm start */
    }
    for (int it = 0; it < K_SOLVER_ITERS; it++) {
        for (int i = 0; i < count; i++) {
            ORow* r = &nrm[i];
            if (r->rhsPen == 0.f) continue;
            const float rv = row_vel(r, b->pushVel, b->turnVel);
            const float imp = solve_lower(r->rhsPen, r->cfm, r->jacInv, rv, r->lower, &r->appliedPush);
            b->pushVel = vadd(b->pushVel, vscale(r->axis, K_CAR_INV_MASS * imp));
            b->turnVel = vadd(b->turnVel, vscale(r->angular, imp));
        }
    }
    for (int it = 0; it < K_SOLVER_ITERS; it++) {
        for (int i = 0; i < count; i++) {
            ORow* r = &nrm[i];
            const float rv = row_vel(r, b->deltaVel, b->deltaAng);
            const float imp = solve_lower(r->rhs, r->cfm, r->jacInv, rv, r->lower, &r->applied);
            row_apply(b, r, imp);
        }
        for (int i = 0; i < count; i++) {
            const float maxImp = fc[i] * nrm[i].applied;
            if (maxImp <= 0.f) continue;
            ORow* r = &fr[i];
            r->lower = -maxImp;
            r->upper = maxImp;
            const float rv = row_vel(r, b->deltaVel, b->deltaAng);
            const float imp = solve_impulse(r->rhs, r->cfm, r->jacInv, rv, r->lower, r->upper, &r->applied);
            row_apply(b, r, imp);
        }
    }
    for (int i = 0; i < count; i++) { pts[i].impulse = nrm[i].applied; pts[i].impulseTan = fr[i].applied; }
}

/* include/Physics/CarArena/Solve.cuh:286-314 */
static void solve_car_arena(OWorld* w, int ci)
{
    OCar* c = &w->cars[ci];
    if (c->demoed) return;
    OBody b = load_body(c);
    apply_suspension(&b, c, w->tickCount);
    OManPoint pts[MAX_MANIFOLD];
    memset(pts, 0, sizeof pts);
    const int count = build_manifold(w, ci, pts);
    if (count > 0) {
        solve_manifold(&b, pts, count);
        if (!(vlensq(b.pushVel) == 0.f && vlensq(b.turnVel) == 0.f)) {
            const V3 splitAng = vscale(b.turnVel, K_SPLIT_TURN_ERP);
            integrate_state(&b.pos, &b.cen, &b.rot, b.pushVel, splitAng);
        }
    }
    c->manCount = count;
    c->manNormal = count > 0 ? pts[0].worldNormal : V_ZERO;
    b.vel = vadd(vadd(b.vel, b.extVel), b.deltaVel);
    b.ang = vadd(vadd(b.ang, b.extAng), b.deltaAng);
    store_body(c, &b);
}

/* ------------------------------------------------------------------ car-car */

typedef struct { V3 cen; Q4 rot; } OBox;
typedef struct { V3 carPosA, carPosB, normal; float depth; } OCC;

static V3 box_axis(const OBox* b, int i) { return qworld(b->rot, v_axis(i)); }

static V3 box_support(const OBox* b, V3 dir)
{
    const V3 ld = qlocal(b->rot, dir);
    const V3 l = v3(copysignf(K_CAR_HALF.x, ld.x), copysignf(K_CAR_HALF.y, ld.y), copysignf(K_CAR_HALF.z, ld.z));
    return vadd(b->cen, qworld(b->rot, l));
}

/* include/Physics/CarCar/SAT.cuh:6-44 */
static void cc_axis(V3 axis, const OBox* A, const OBox* B, int idx, OSat* r)
{
    const float l = vlensq(axis);
    if (l < 1e-12f) return;
    axis = vscale(axis, o_rsqrt(l));
    const float rA = vdot(vabs(qlocal(A->rot, axis)), K_CAR_HALF);
    const float cA = vdot(A->cen, axis);
    const float rB = vdot(vabs(qlocal(B->rot, axis)), K_CAR_HALF);
    const float cB = vdot(B->cen, axis);
    const float aMin = cA - rA, aMax = cA + rA, bMin = cB - rB, bMax = cB + rB;
    if (aMax < bMin || bMax < aMin) { r->overlap = 0; return; }
    const float dAB = aMax - bMin, dBA = bMax - aMin;
    const float depth = o_min(dAB, dBA);
    if (depth * (idx >= 6 ? 1.05f : 1.f) >= r->minPen) return;
    r->minPen = depth;
    r->minAxis = dAB < dBA ? vneg(axis) : axis;
    r->axisIdx = idx;
}

/* include/Physics/CarCar/SAT.cuh:46-125 */
static OSat cc_sat(const OBox* A, const OBox* B)
{
    OSat r = { 1, 0, K_FLT_MAX, { 0.f, 0.f, 0.f } };
    V3 aa[3], ba[3];
    for (int i = 0; i < 3; i++) { aa[i] = box_axis(A, i); ba[i] = box_axis(B, i); }
    const V3 delta = vsub(vscale(B->cen, .02f), vscale(A->cen, .02f));
    const V3 half = vscale(K_CAR_HALF, .02f);
    float al[3][3];
    for (int i = 0; i < 3; i++) for (int j = 0; j < 3; j++) al[i][j] = fabsf(vdot(aa[i], ba[j]));
    for (int i = 0; i < 3; i++) {
        const float dist = vdot(delta, aa[i]);
        const float rad = vget(half, i) + half.x * al[i][0] + half.y * al[i][1] + half.z * al[i][2];
        const float depth = (rad - fabsf(dist)) * 50.f;
        if (depth < 0.f) { r.overlap = 0; return r; }
        if (depth < r.minPen) { r.minPen = depth; r.minAxis = dist > 0 ? vneg(aa[i]) : aa[i]; r.axisIdx = i; }
    }
    for (int i = 0; i < 3; i++) {
        const float dist = vdot(delta, ba[i]);
        const float rad = half.x * al[0][i] + half.y * al[1][i] + half.z * al[2][i] + vget(half, i);
        const float depth = (rad - fabsf(dist)) * 50.f;
        if (depth < 0.f) { r.overlap = 0; return r; }
        if (depth < r.minPen) { r.minPen = depth; r.minAxis = dist > 0 ? vneg(ba[i]) : ba[i]; r.axisIdx = 3 + i; }
    }
    for (int i = 0; i < 3; i++)
        for (int j = 0; j < 3; j++) {
            cc_axis(vcross(aa[i], ba[j]), A, B, 6 + i * 3 + j, &r);
            if (!r.overlap) return r;
        }
    return r;
}

/* include/Physics/CarCar/Clip.cuh:25-197 */
static int cc_contacts(const OSat* s, const OBox* A, const OBox* B, OCC* out)
{
    if (s->axisIdx >= 6) {
        const V3 pA = box_support(A, vneg(s->minAxis));
        const V3 pB = box_support(B, s->minAxis);
        out[0].carPosA = qlocal(A->rot, vsub(pA, A->cen));
        out[0].carPosB = qlocal(B->rot, vsub(pB, B->cen));
        out[0].normal = s->minAxis;
        out[0].depth = s->minPen;
        return 1;
    }
    const int refIsA = s->axisIdx < 3;
    const OBox* ref = refIsA ? A : B;
    const OBox* inc = refIsA ? B : A;
    const int faxis = refIsA ? s->axisIdx : s->axisIdx - 3;
    V3 refN = box_axis(ref, faxis);
    if (vdot(refN, vsub(inc->cen, ref->cen)) < 0.f) refN = vneg(refN);

    /* incident face of the other box */
    int iaxis = 0;
    V3 inorm = V_ZERO;
    float bestAl = -1.f;
    for (int a = 0; a < 3; a++) {
        const V3 n = box_axis(inc, a);
        const float d = vdot(n, refN);
        const float al = fabsf(d);
        if (al <= bestAl) continue;
        bestAl = al; iaxis = a; inorm = d > 0.f ? vneg(n) : n;
    }
    const int au = (iaxis + 1) % 3, av = (iaxis + 2) % 3;
    const V3 eu = vscale(box_axis(inc, au), vget(K_CAR_HALF, au));
    const V3 ev = vscale(box_axis(inc, av), vget(K_CAR_HALF, av));
    const V3 center = vadd(inc->cen, vscale(inorm, vget(K_CAR_HALF, iaxis)));
    V3 bufA[8], bufB[8];
    bufA[0] = vsub(vsub(center, eu), ev);
    bufA[1] = vsub(vadd(center, eu), ev);
    bufA[2] = vadd(vadd(center, eu), ev);
    bufA[3] = vadd(vsub(center, eu), ev);
    V3* in = bufA; V3* o = bufB;
    int cnt = 4;
    for (int a = 0; a < 3 && cnt > 0; a++) {
        if (a == faxis) continue;
        const V3 side = box_axis(ref, a);
        const float ext = vget(K_CAR_HALF, a);
        const float maxD = vdot(ref->cen, side) + ext;
        const float minD = vdot(ref->cen, vneg(side)) + ext;
        cnt = clip_plane(in, cnt, o, side, maxD);
        { V3* sw = in; in = o; o = sw; }
        if (cnt == 0) break;
        cnt = clip_plane(in, cnt, o, vneg(side), minD);
        { V3* sw = in; in = o; o = sw; }
    }
    const V3 refCenter = vadd(ref->cen, vscale(refN, vget(K_CAR_HALF, faxis)));
    int n = 0;
    for (int i = 0; i < cnt && n < MAX_MANIFOLD; i++) {
        const float depth = vdot(vsub(refCenter, in[i]), refN);
        if (depth < -K_CONTACT_BREAK) continue;
        const V3 onRef = vadd(in[i], vscale(refN, depth));
        const V3 pA = refIsA ? onRef : in[i];
        const V3 pB = !refIsA ? onRef : in[i];
        out[n].carPosA = qlocal(A->rot, vsub(pA, A->cen));
        out[n].carPosB = qlocal(B->rot, vsub(pB, B->cen));
        out[n].normal = s->minAxis;
        out[n].depth = o_max(depth, 0.f);
        n++;
    }
    if (n > 0) return n;
    out[0].carPosA = qlocal(A->rot, vsub(refCenter, A->cen));
    out[0].carPosB = qlocal(B->rot, vsub(refCenter, B->cen));
    out[0].normal = s->minAxis;
    out[0].depth = s->minPen;
    return 1;
}

typedef struct {
    V3 axis, relCrossA, relCrossB, angularA, angularB;
    float jacInv, rhs, rhsPen, applied, appliedPush;
} OPRow;

static OPRow pair_axis_row(const OBody* A, const OBody* B, V3 axis, V3 relA, V3 relB)
{
    OPRow r;
    memset(&r, 0, sizeof r);
    r.axis = axis;
    r.relCrossA = vcross(relA, axis);
    r.relCrossB = vcross(relB, axis);
    r.angularA = inv_inertia_world(A->rot, r.relCrossA);
    r.angularB = inv_inertia_world(B->rot, r.relCrossB);
    const float denom = 2.f * K_CAR_INV_MASS + vdot(axis, vcross(r.angularA, relA)) + vdot(axis, vcross(r.angularB, relB));
    r.jacInv = 1.f / o_max(denom, 1e-8f);
    return r;
}

static float pair_vel(const OPRow* r, V3 lA, V3 aA, V3 lB, V3 aB)
{
    return vdot(r->axis, lA) + vdot(r->relCrossA, aA) - vdot(r->axis, lB) - vdot(r->relCrossB, aB);
}

static void pair_apply(OBody* A, OBody* B, const OPRow* r, float imp, int split)
{
    V3* lA = split ? &A->pushVel : &A->deltaVel;
    V3* aA = split ? &A->turnVel : &A->deltaAng;
    V3* lB = split ? &B->pushVel : &B->deltaVel;
    V3* aB = split ? &B->turnVel : &B->deltaAng;
    *lA = vadd(*lA, vscale(r->axis, K_CAR_INV_MASS * imp));
    *aA = vadd(*aA, vscale(r->angularA, imp));
    *lB = vsub(*lB, vscale(r->axis, K_CAR_INV_MASS * imp));
    *aB = vsub(*aB, vscale(r->angularB, imp));
}

/* include/Physics/CarCar/Solver.cuh:187-244 */
static void pair_solve(OBody* A, OBody* B, const OCC* cts, int count, float* impN, float* impT)
{
    OPRow nr[MAX_MANIFOLD], fr[MAX_MANIFOLD];
    for (int i = 0; i < count; i++) {
        const V3 relA = vadd(vsub(A->cen, A->pos), qworld(A->rot, cts[i].carPosA));
        const V3 relB = vadd(vsub(B->cen, B->pos), qworld(B->rot, cts[i].carPosB));
        OPRow n = pair_axis_row(A, B, cts[i].normal, relA, relB);
        const float rv = pair_vel(&n, A->vel, A->ang, B->vel, B->ang);
        const float bounce = rv < -K_RESTITUTION_VEL_THRESH ? K_CARCAR_RESTITUTION * -rv : 0.f;
        const float pen = o_max(cts[i].depth - K_LINEAR_SLOP, 0.f);
        n.rhs = (bounce - rv) * n.jacInv;
        n.rhsPen = pen * K_CONTACT_ERP / K_DT * n.jacInv;
        nr[i] = n;
        const V3 vA = vadd(A->vel, vcross(A->ang, relA));
        const V3 vB = vadd(B->vel, vcross(B->ang, relB));
        const V3 rel = vsub(vA, vB);
        const float nv = vdot(cts[i].normal, rel);
        V3 tan = vsub(rel, vscale(cts[i].normal, nv));
        const float tl = vlensq(tan);
        const float thr = o_max(K_FLT_EPS, nv * nv * 1e-8f);
        tan = tl > thr ? vscale(tan, o_rsqrt(tl)) : fallback_tangent(cts[i].normal);
        OPRow t = pair_axis_row(A, B, tan, relA, relB);
        const float tv = pair_vel(&t, A->vel, A->ang, B->vel, B->ang);
        t.rhs = -tv * t.jacInv;
        fr[i] = t;
    }
    for (int it = 0; it < K_SOLVER_ITERS; it++)
        for (int i = 0; i < count; i++) {
            OPRow* r = &nr[i];
            const float rv = pair_vel(r, A->pushVel, A->turnVel, B->pushVel, B->turnVel);
            const float imp = solve_lower(r->rhsPen, 0.f, r->jacInv, rv, 0.f, &r->appliedPush);
            pair_apply(A, B, r, imp, 1);
        }
    for (int it = 0; it < K_SOLVER_ITERS; it++) {
        for (int i = 0; i < count; i++) {
            OPRow* r = &nr[i];
            const float rv = pair_vel(r, A->deltaVel, A->deltaAng, B->deltaVel, B->deltaAng);
            const float imp = solve_lower(r->rhs, 0.f, r->jacInv, rv, 0.f, &r->applied);
            pair_apply(A, B, r, imp, 0);
        }
        for (int i = 0; i < count; i++) {
            const float maxImp = K_CARCAR_FRICTION * nr[i].applied;
            if (maxImp <= 0.f) continue;
            OPRow* r = &fr[i];
            const float rv = pair_vel(r, A->deltaVel, A->deltaAng, B->deltaVel, B->deltaAng);
            const float imp = solve_impulse(r->rhs, 0.f, r->jacInv, rv, -maxImp, maxImp, &r->applied);
            pair_apply(A, B, r, imp, 0);
        }
    }
    for (int i = 0; i < count; i++) { impN[i] = nr[i].applied; impT[i] = fr[i].applied; }
}

static float bump_curve(float s, float lo, float mid, float hi)
{
    if (s <= 0.f) return lo;
    if (s <= 1400.f) return lo + (mid - lo) * (s / 1400.f);
    if (s <= 2200.f) return mid + (hi - mid) * ((s - 1400.f) / 800.f);
    return hi;
}

/* include/Physics/CarCar/Response.cuh:59-74 */
static int front_hit(const OCC* cts, int count, int aIsBumper, V3 delta, Q4 bumperRot)
{
    if (qlocal(bumperRot, delta).x > K_BUMP_MIN_FWD) return 1;
    for (int i = 0; i < count; i++) {
        const V3 p = aIsBumper ? cts[i].carPosA : cts[i].carPosB;
        if (p.x + K_CAR_OFFSETS.x > K_BUMP_MIN_FWD) return 1;
    }
    return 0;
}

/* include/Physics/CarCar/Solve.cuh:63-151 and Response.cuh:76-192 */
static void car_car_pair(OWorld* w, int ia, int ib)
{
    OCar* ca = &w->cars[ia];
    OCar* cb = &w->cars[ib];
    if (ca->demoed || cb->demoed) return;
    OBox A = { ca->cen, ca->rot }, B = { cb->cen, cb->rot };
    const V3 cd = vsub(B.cen, A.cen);
    const float maxDist = 2.f * vlen(K_CAR_HALF);
    if (vlensq(cd) > maxDist * maxDist) return;
    const OSat s = cc_sat(&A, &B);
    if (!s.overlap) return;
    OCC cts[MAX_MANIFOLD];
    const int count = cc_contacts(&s, &A, &B, cts);
    if (count == 0) return;

    /* findDemo, on the pre-solve state */
    int demoBumper = -1, demoVictim = -1;
    {
        const int teamA = (ia % w->nCars) < w->nBlue ? 0 : 1;
        const int teamB = (ib % w->nCars) < w->nBlue ? 0 : 1;
        if (teamA != teamB && !(s.minPen < 5.f)) {
            for (int side = 0; side < 2; side++) {
                const int aB = side == 0;
                const int bumper = aB ? ia : ib, victim = aB ? ib : ia;
                const V3 bv = w->cars[bumper].vel, vv = w->cars[victim].vel;
                const V3 bp = w->cars[bumper].pos, vp = w->cars[victim].pos;
                const Q4 br = aB ? A.rot : B.rot;
                const float speed = vlen(bv);
                if (speed < K_SUPERSONIC) continue;
                const V3 delta = vsub(vp, bp);
                if (vdot(bv, delta) <= 0.f) continue;
                const V3 velDir = vdivs(bv, speed);
                const V3 hitDir = vnorm(delta);
                const float closing = vdot(bv, hitDir);
                if (closing <= vdot(vv, velDir)) continue;
                if (!front_hit(cts, count, aB, delta, br)) continue;
                demoBumper = bumper; demoVictim = victim;
                break;
            }
        }
    }

    OBody bA = load_body(ca), bB = load_body(cb);
    const V3 preA = bA.vel, preB = bB.vel;
    float impN[MAX_MANIFOLD], impT[MAX_MANIFOLD];
    pair_solve(&bA, &bB, cts, count, impN, impT);

    /* applyPairResult */
    bA.vel = vadd(bA.vel, bA.deltaVel); bA.ang = vadd(bA.ang, bA.deltaAng);
    bB.vel = vadd(bB.vel, bB.deltaVel); bB.ang = vadd(bB.ang, bB.deltaAng);
    bA.pos = vadd(bA.pos, vscale(bA.pushVel, K_DT));
    bB.pos = vadd(bB.pos, vscale(bB.pushVel, K_DT));
    bA.rot = ophys_integrate_quat(bA.rot, vscale(bA.turnVel, K_SPLIT_TURN_ERP));
    bB.rot = ophys_integrate_quat(bB.rot, vscale(bB.turnVel, K_SPLIT_TURN_ERP));
    bA.cen = vadd(bA.pos, qworld(bA.rot, K_CAR_OFFSETS));
    bB.cen = vadd(bB.pos, qworld(bB.rot, K_CAR_OFFSETS));
    clamp_body(&bA); clamp_body(&bB);
    store_body(ca, &bA); store_body(cb, &bB);

    if (demoVictim >= 0) {
        OCar* v = &w->cars[demoVictim];
        V3 pos = v->pos, cen;
        Q4 rot = v->rot;
        integrate_state(&pos, &cen, &rot, v->vel, v->ang);
        v->pos = pos; v->cen = cen; v->rot = rot;
        v->demoed = 1;
        v->demoTimer = K_DEMO_RESPAWN_TIME + K_DT;
        w->cars[demoBumper].contactIdx = demoVictim;
        w->cars[demoBumper].contactCooldown = K_BUMP_COOLDOWN;
        const uint32_t seed = (uint32_t)w->seed ^ (uint32_t)demoVictim * 0x9e3779b9u ^ (uint32_t)w->tickCount;
        v->in.respawnIdx = o_random_index(seed, 4);
        v->in.lastRespawnDir = 0;
        return;
    }

    /* tryApplyBump, A as bumper then B */
    for (int side = 0; side < 2; side++) {
        const int aB = side == 0;
        const int bumper = aB ? ia : ib, victim = aB ? ib : ia;
        const V3 bv = aB ? preA : preB, vv = aB ? preB : preA;
        const V3 bp = aB ? bA.pos : bB.pos, vp = aB ? bB.pos : bA.pos;
        const Q4 br = aB ? bA.rot : bB.rot, vr = aB ? bB.rot : bA.rot;
        if (w->cars[bumper].contactIdx == victim && w->cars[bumper].contactCooldown > 0.f) continue;
        const V3 delta = vsub(vp, bp);
        if (vdot(bv, delta) <= 0.f) continue;
        const float speed = vlen(bv);
        if (speed < 1e-6f) continue;
        const V3 velDir = vdivs(bv, speed);
        const V3 hitDir = vnorm(delta);
        const float closing = vdot(bv, hitDir);
        if (closing <= vdot(vv, velDir)) continue;
        if (!front_hit(cts, count, aB, delta, br)) continue;
        const int grounded = w->cars[victim].in.onGround != 0;
        const float fwdScale = grounded ? bump_curve(closing, 5.f / 6.f, 1100.f, 1530.f)
                                        : bump_curve(closing, 5.f / 6.f, 1390.f, 1945.f);
        const V3 up = grounded ? qworld(vr, V_Z) : V_Z;
        const V3 imp = vadd(vscale(velDir, fwdScale), vscale(up, bump_curve(closing, 2.f / 6.f, 278.f, 417.f)));
        w->cars[victim].imp = vadd(w->cars[victim].imp, imp);
        w->cars[bumper].contactIdx = victim;
        w->cars[bumper].contactCooldown = K_BUMP_COOLDOWN;
    }
}

/* ------------------------------------------------------------- ball vs arena */

typedef struct { V3 point, relPos, normal; float depth; int tri; V3 reductionPos; } OBallContact;

/* include/Physics/BallArena/Contact.cuh:204-251 (Ericson, RTCD 5.1.5) */
static V3 closest_on_triangle(V3 p, V3 a, V3 b, V3 c)
{
    const V3 ab = vsub(b, a), ac = vsub(c, a);
    const V3 ap = vsub(p, a);
    const float abAp = vdot(ab, ap), acAp = vdot(ac, ap);
    if (abAp <= 0.f && acAp <= 0.f) return a;
    const V3 bp = vsub(p, b);
    const float abBp = vdot(ab, bp), acBp = vdot(ac, bp);
    if (abBp >= 0.f && acBp <= abBp) return b;
    const float wc = abAp * acBp - abBp * acAp;
    if (wc <= 0.f && abAp >= 0.f && abBp <= 0.f) return vadd(a, vscale(ab, abAp / (abAp - abBp)));
    const V3 cp = vsub(p, c);
    const float abCp = vdot(ab, cp), acCp = vdot(ac, cp);
    if (acCp >= 0.f && abCp <= acCp) return c;
    const float wb = abCp * acAp - abAp * acCp;
    if (wb <= 0.f && acAp >= 0.f && acCp <= 0.f) return vadd(a, vscale(ac, acAp / (acAp - acCp)));
    const float wa = abBp * acCp - abCp * acBp;
    if (wa <= 0.f && acBp >= abBp && abCp >= acCp) {
        const float e = acBp - abBp;
        return vadd(b, vscale(vsub(c, b), e / (e + abCp - acCp)));
    }
    const float inv = 1.f / (wa + wb + wc);
    return vadd(vadd(a, vscale(ab, wb * inv)), vscale(ac, wc * inv));
}

/* include/Physics/BallArena/Contact.cuh:253-290 */
static int sphere_triangle(OBallContact* ct, V3 center, float radius, V3 t0, V3 t1, V3 t2)
{
    const V3 point = closest_on_triangle(center, t0, t1, t2);
    const V3 delta = vsub(center, point);
    const float dsq = vlensq(delta);
    const float cr = radius + K_BALL_ARENA_BREAK;
    if (dsq >= cr * cr) return 0;
    V3 n = vcross(vsub(t1, t0), vsub(t2, t0));
    const float nl = vlensq(n);
    if (nl < 1e-12f) return 0;
    n = vscale(n, o_rsqrt(nl));
    if (dsq > 1e-8f && vdot(n, delta) < 0.f) n = vneg(n);
    if (dsq > 1e-8f) n = vscale(delta, o_rsqrt(dsq));
    ct->point = point;
    ct->relPos = vscale(n, -radius);
    ct->normal = n;
    ct->depth = dsq > 1e-8f ? radius - sqrtf(dsq) : radius;
    return 1;
}

/* include/Physics/BallArena/Contact.cuh:345-394 */
static int ball_replacement(const OBallContact* cs, const OBallContact* cand)
{
    int deepest = -1;
    float depth = cand->depth;
    for (int i = 0; i < 4; i++) if (cs[i].depth > depth) { deepest = i; depth = cs[i].depth; }
    float a[4] = { 0.f, 0.f, 0.f, 0.f };
    const V3 p = cand->reductionPos;
    if (deepest != 0) a[0] = vlensq(vcross(vsub(p, cs[1].reductionPos), vsub(cs[3].reductionPos, cs[2].reductionPos)));
    if (deepest != 1) a[1] = vlensq(vcross(vsub(p, cs[0].reductionPos), vsub(cs[3].reductionPos, cs[2].reductionPos)));
    if (deepest != 2) a[2] = vlensq(vcross(vsub(p, cs[0].reductionPos), vsub(cs[3].reductionPos, cs[1].reductionPos)));
    if (deepest != 3) a[3] = vlensq(vcross(vsub(p, cs[0].reductionPos), vsub(cs[2].reductionPos, cs[1].reductionPos)));
    int best = 0;
    for (int i = 1; i < 4; i++) if (a[i] > a[best]) best = i;
    return best;
}

/* include/Physics/BallArena/Contact.cuh:86-159 */
static void adjust_ball_edge(OBallContact* ct, V3 point, V3 t0, V3 t1, V3 t2, V3 angles)
{
    const V3 vs[3] = { t0, t1, t2 };
    int bestEdge = -1;
    float bestSq = 25.f;
    for (int e = 0; e < 3; e++) {
        if (fabsf(vget(angles, e)) >= K_BOUNDARY_EDGE_ANGLE) continue;
        const V3 s = vs[e], en = vs[(e + 1) % 3];
        const V3 edge = vsub(en, s);
        const float t = o_clamp(vdot(vsub(point, s), edge) / vlensq(edge), 0.f, 1.f);
        const V3 nearest = vadd(s, vscale(edge, t));
        const float sq = vlensq(vsub(point, nearest));
        if (sq < bestSq) { bestSq = sq; bestEdge = e; }
    }
    if (bestEdge < 0) return;
    const V3 face = vnorm(vcross(vsub(t1, t0), vsub(t2, t0)));
    const float angle = vget(angles, bestEdge);
    if (angle == 0.f) {
        if (vdot(face, ct->normal) >= 0.f) ct->normal = face;
        return;
    }
    const float side = angle > 0.f ? 1.f : -1.f;
    const V3 edgeAxis = vnorm(vsub(vs[(bestEdge + 1) % 3], vs[bestEdge]));
    const V3 nA = vscale(face, side);
    const V3 nB = vscale(o_rotate_axis(face, edgeAxis, angle), side);
    if (vdot(ct->normal, nA) < 0.f && vdot(ct->normal, nB) < 0.f) {
        if (vdot(face, ct->normal) >= 0.f) ct->normal = face;
        return;
    }
    V3 cl;
    if (clamp_normal(edgeAxis, nA, ct->normal, angle, &cl) && vdot(cl, face) > 0.f) ct->normal = vnorm(cl);
}

/* include/Physics/BallArena/Contact.cuh:292-343: the sphere against one
 * native triangle, centre and vertices in Bullet units */
static int native_sphere_triangle(OBallContact* ct, V3 center, V3 t0, V3 t1, V3 t2)
{
    const float radius = K_BALL_RADIUS * .02f;
    const float extent = radius + K_BALL_ARENA_BREAK * .02f;
    const V3 e01 = vsub(t1, t0), e02 = vsub(t2, t0), off = vsub(center, t0);
    const V3 face = vcross(e01, e02);
    const float nl = vlensq(face);
    if (nl < 1e-14f) return 0;
    V3 n = vscale(face, 1.f / sqrtf(nl));
    float plane = vdot(off, n);
    if (plane < 0.f) { plane = -plane; n = vneg(n); }
    if (plane >= extent) return 0;
    const float gamma = vdot(vcross(e01, off), face) / nl;
    const float beta = vdot(vcross(off, e02), face) / nl;
    const float alpha = 1.f - gamma - beta;
    const int inside = alpha >= 0.f && alpha <= 1.f && beta >= 0.f && beta <= 1.f && gamma >= 0.f && gamma <= 1.f;
    ct->point = inside ? vsub(center, vscale(n, plane)) : closest_on_triangle(center, t0, t1, t2);
    const V3 delta = vsub(center, ct->point);
    const float dsq = vlensq(delta);
    if (dsq >= extent * extent) return 0;
    const float dist = sqrtf(dsq);
    ct->normal = dsq > K_FLT_EPS ? vscale(delta, 1.f / dist) : n;
    ct->depth = dsq > K_FLT_EPS ? radius - dist : radius;
    ct->relPos = vsub(vsub(ct->point, vscale(ct->normal, ct->depth)), center);
    ct->reductionPos = ct->relPos;
    return 1;
}

/* include/Physics/BallArena/Contact.cuh:161-202: the native internal-edge
 * correction, sides chosen by the metadata flags (bit e: face side of edge e,
 * bit e + 3: the neighbour's normal reversed) */
static void adjust_native_ball_edge(OBallContact* ct, V3 t0, V3 t1, V3 t2, V3 angles, int flags, float edgeDistance)
{
    const V3 vs[3] = { t0, t1, t2 };
    int best = -1;
    float bestSq = edgeDistance * edgeDistance;
    for (int e = 0; e < 3; e++) {
        if (fabsf(vget(angles, e)) >= K_BOUNDARY_EDGE_ANGLE) continue;
        const V3 st = vs[e], en = vs[(e + 1) % 3];
        const V3 edge = vsub(en, st);
        const float t = o_clamp(vdot(vsub(ct->point, st), edge) / vlensq(edge), 0.f, 1.f);
        const float sq = vlensq(vsub(ct->point, vadd(st, vscale(edge, t))));
        if (sq < bestSq) { bestSq = sq; best = e; }
    }
    if (best < 0) return;
    const V3 face = vnorm(vcross(vsub(t1, t0), vsub(t2, t0)));
    const V3 edgeDir = vnorm(vsub(vs[best], vs[(best + 1) % 3]));
    const float angle = vget(angles, best);
    int concave = angle == 0.f;
    if (!concave) {
        const float sign = (flags & (1 << best)) ? 1.f : -1.f;
        V3 other = o_rotate_axis(face, edgeDir, angle);
        if (flags & (1 << (best + 3))) other = vneg(other);
        concave = vdot(ct->normal, vscale(face, sign)) < 0.f && vdot(ct->normal, vscale(other, sign)) < 0.f;
        if (!concave) {
            V3 cl;
            if (clamp_normal(edgeDir, vscale(face, sign), ct->normal, angle, &cl) && vdot(cl, face) > 0.f)
                ct->normal = cl;
        }
    }
    if (concave && vdot(face, ct->normal) >= 0.f) ct->normal = face;
}

/* the arena planes of the native branch: floor, ceiling, side walls */
static const V3 k_plane_normals[4] = { { 0.f, 0.f, 1.f }, { 0.f, 0.f, -1.f }, { 1.f, 0.f, 0.f }, { -1.f, 0.f, 0.f } };
static const float k_plane_offsets[4] = { 0.f, -2044.f, -4096.f, -4096.f };

static float native_plane_depth(V3 center, int p)
{
    return K_BALL_RADIUS - (vdot(k_plane_normals[p], center) - k_plane_offsets[p]);
}

static int count_native_planes(V3 center)
{
    int n = 0;
    for (int p = 0; p < 4; p++) n += native_plane_depth(center, p) > -K_BALL_ARENA_BREAK;
    return n;
}

/* include/Physics/BallArena/Contact.cuh:478-511: native contacts back to
 * Unreal units, then the four arena planes as analytic contacts */
static int finish_native_ball_contacts(OBallContact* cs, int count, V3 center)
{
    const V3* normals = k_plane_normals;
    for (int i = 0; i < count; i++) {
        cs[i].point = vscale(cs[i].point, 50.f);
        cs[i].relPos = vscale(cs[i].relPos, 50.f);
        cs[i].depth *= 50.f;
    }
    for (int p = 0; p < 4; p++) {
        const float depth = native_plane_depth(center, p);
        if (depth > -K_BALL_ARENA_BREAK) {
            OBallContact* c = &cs[count++];
            memset(c, 0, sizeof *c);
            c->point = vsub(center, vscale(normals[p], K_BALL_RADIUS - depth));
            c->relPos = vscale(normals[p], -K_BALL_RADIUS);
            c->normal = normals[p];
            c->depth = depth;
            c->tri = -1;
        }
    }
    return count;
}

/* include/Physics/BallArena/Contact.cuh:513-594: the cells' ball lists merged
 * in order (by triangle index, or with native metadata by (order key,
 * triangle)), each distinct triangle once; at most four contacts kept per
 * native mesh.  With metadata a contact that would need a slot past the 68
 * less the planes in reach is dropped: the reference writes past its array
 * there. */
static int gather_ball_contacts(const OArena* A, V3 center, OBallContact* cs)
{
    const int native = A->native;
    const int* lists = native ? A->ballTris : A->cellTris;
    const float ext = K_BALL_RADIUS + K_BALL_ARENA_BREAK;
    int lo[3], hi[3];
    oarena_cell3(vsubs(center, ext), &lo[0], &lo[1], &lo[2]);
    oarena_cell3(vadds(center, ext), &hi[0], &hi[1], &hi[2]);
    int cursor[27], end[27], cells = 0;
    for (int z = lo[2]; z <= hi[2]; z++)
        for (int y = lo[1]; y <= hi[1]; y++)
            for (int x = lo[0]; x <= hi[0]; x++) {
                const int c = oarena_flat(x, y, z);
                cursor[cells] = A->cellPrefix[c];
                end[cells] = A->cellPrefix[c + 1];
                cells++;
            }
    int count = 0, mesh = -1, base = 0, localCount = 0, lastTri = -1;
    int room = MAX_BALL_CONTACTS;
    if (native) room -= count_native_planes(center);
    for (;;) {
        int sel = -1, tri = -1;
        long long key = 0x7fffffffffffffffLL;
        for (int c = 0; c < cells; c++) {
            if (cursor[c] >= end[c]) continue;
            const int t = lists[cursor[c]];
            const long long k = native ? (long long)A->nkey[t] * 4294967296LL + t : t;
            if (k < key) { key = k; sel = c; tri = t; }
        }
        if (sel >= 0) cursor[sel]++;
        if (tri < 0) break;
        if (tri == lastTri) continue;
        lastTri = tri;
        const int current = native ? A->nmesh[tri] : 0;
        if (native && current < 0) continue;
        OBallContact ct;
        memset(&ct, 0, sizeof ct);
        ct.tri = -1;
        V3 t0, t1, t2;
        if (native) {
            t0 = A->nverts[3 * tri]; t1 = A->nverts[3 * tri + 1]; t2 = A->nverts[3 * tri + 2];
            if (!native_sphere_triangle(&ct, vscale(center, .02f), t0, t1, t2)) continue;
        } else {
            t0 = A->verts[A->tris[3 * tri]]; t1 = A->verts[A->tris[3 * tri + 1]]; t2 = A->verts[A->tris[3 * tri + 2]];
            if (!sphere_triangle(&ct, center, K_BALL_RADIUS, t0, t1, t2)) continue;
            ct.reductionPos = ct.relPos;
        }
        ct.tri = tri;
        if (current != mesh) { base = count; localCount = 0; mesh = current; }
        int slot;
        if (localCount < 4) {
            if (count == room) continue;
            slot = localCount++;
            count++;
        }
        else slot = ball_replacement(cs + base, &ct);
        if (native) {
            adjust_native_ball_edge(&ct, t0, t1, t2, A->nangs[tri], A->nflags[tri], .1f);
            ct.point = vadd(vadd(vscale(center, .02f), ct.relPos), vscale(ct.normal, ct.depth));
        } else {
            adjust_ball_edge(&ct, ct.point, t0, t1, t2, A->angs[tri]);
            ct.point = vadd(vadd(center, ct.relPos), vscale(ct.normal, ct.depth));
        }
        cs[base + slot] = ct;
    }
    return native ? finish_native_ball_contacts(cs, count, center) : count;
}

typedef struct { V3 pos, vel, velNoExt, ang, deltaVel, deltaAng, pushVel, pushAng; } OBallBody;
typedef struct { V3 axis, relCross; float jacInv, rhs, rhsPen, applied, appliedPush, lower, upper; } OBRow;

static OBRow ball_axis_row(V3 axis, V3 relPos)
{
    OBRow r;
    memset(&r, 0, sizeof r);
    r.axis = axis;
    r.relCross = vcross(relPos, axis);
    const float denom = K_BALL_INV_MASS + K_BALL_INV_INERTIA * vlensq(r.relCross);
    r.jacInv = 1.f / o_max(denom, 1e-8f);
    r.upper = 1e10f;
    return r;
}

static float brow_vel(const OBRow* r, V3 lin, V3 ang) { return vdot(r->axis, lin) + vdot(r->relCross, ang); }

static OBRow ball_normal_row(const OBallBody* b, V3 normal, float depth, V3 relPos, int split)
{
    OBRow r = ball_axis_row(normal, relPos);
    const float rv = brow_vel(&r, b->vel, b->ang);
    const float restv = brow_vel(&r, b->velNoExt, b->ang);
    float bounce = fabsf(restv) >= K_RESTITUTION_VEL_THRESH ? K_BALL_RESTITUTION * -restv : 0.f;
    bounce = o_max(bounce, 0.f);
    const float posErr = o_max(depth, 0.f) * K_CONTACT_ERP / K_DT;
    const float posImp = posErr * r.jacInv;
    const float velImp = (bounce - rv) * r.jacInv;
    if (!split) r.rhs = velImp;
    else if (-depth > K_SPLIT_PEN_THRESH) r.rhs = posImp + velImp;
    else { r.rhs = velImp; r.rhsPen = posImp; }
    return r;
}

static void ball_apply(OBallBody* b, const OBRow* r, float imp, int split)
{
    V3* lin = split ? &b->pushVel : &b->deltaVel;
    V3* ang = split ? &b->pushAng : &b->deltaAng;
    *lin = vadd(*lin, vscale(r->axis, K_BALL_INV_MASS * imp));
    *ang = vadd(*ang, vscale(r->relCross, K_BALL_INV_INERTIA * imp));
}

/* include/Physics/BallArena/Solver.cuh:197-258 */
static void solve_ball_contacts(OBallBody* b, const OBallContact* cs, int count, int ballWasHit)
{
    if (count == 0) return;
    OBRow split[MAX_BALL_CONTACTS];
    V3 totalN = V_ZERO;
    float totalR = 0.f;
    const int doSplit = !ballWasHit || count != 1 || cs[0].normal.z < 0.999f;
    for (int i = 0; i < count; i++) {
        split[i] = ball_normal_row(b, cs[i].normal, cs[i].depth, cs[i].relPos, doSplit);
        totalN = vadd(totalN, cs[i].normal);
        totalR += sqrtf(vlensq(cs[i].relPos));
    }
    const V3 avgN = vscale(totalN, 1.f / (float)count);
    const V3 avgRel = vscale(avgN, -totalR / (float)count);
    const float avgDepth = -totalR / (float)count;
    OBRow nr = ball_normal_row(b, avgN, avgDepth, avgRel, 0);
    /* friction row */
    const V3 pv = vadd(b->vel, vcross(b->ang, avgRel));
    const float nv = vdot(avgN, pv);
    V3 tan = vsub(pv, vscale(avgN, nv));
    const float tl = vlensq(tan);
    tan = tl > 1e-8f ? vscale(tan, o_rsqrt(tl)) : fallback_tangent(avgN);
    OBRow fr = ball_axis_row(tan, avgRel);
    fr.rhs = -brow_vel(&fr, b->vel, b->ang) * fr.jacInv;
    fr.upper = 0.f;

    for (int it = 0; it < K_SOLVER_ITERS; it++)
        for (int i = 0; i < count; i++) {
            OBRow* r = &split[i];
            if (r->rhsPen == 0.f) continue;
            const float rv = brow_vel(r, b->pushVel, b->pushAng);
            const float imp = solve_lower(r->rhsPen, 0.f, r->jacInv, rv, r->lower, &r->appliedPush);
            ball_apply(b, r, imp, 1);
        }
    for (int it = 0; it < K_SOLVER_ITERS; it++) {
        {
            const float rv = brow_vel(&nr, b->deltaVel, b->deltaAng);
            const float imp = solve_lower(nr.rhs, 0.f, nr.jacInv, rv, nr.lower, &nr.applied);
            ball_apply(b, &nr, imp, 0);
        }
        const float maxImp = K_BALL_FRICTION * nr.applied;
        if (maxImp > 0.f) {
            const float rv = brow_vel(&fr, b->deltaVel, b->deltaAng);
            const float imp = solve_impulse(fr.rhs, 0.f, fr.jacInv, rv, -maxImp, maxImp, &fr.applied);
            ball_apply(b, &fr, imp, 0);
        }
    }
    b->vel = vadd(b->vel, b->deltaVel);
    b->ang = vadd(b->ang, b->deltaAng);
    const float ss = vlensq(b->vel);
    if (ss > K_BALL_MAX_SPEED * K_BALL_MAX_SPEED) b->vel = vscale(b->vel, K_BALL_MAX_SPEED * o_rsqrt(ss));
    const float as = vlensq(b->ang);
    if (as > K_BALL_MAX_ANG * K_BALL_MAX_ANG) b->ang = vscale(b->ang, K_BALL_MAX_ANG * o_rsqrt(as));
}

/* Test probe: the ball-arena contacts gathered for a ball centred at
 * `center`, in slot order: triangle, contact point, normal (after the
 * internal-edge adjustment), depth, and the pre-adjustment offset from the
 * centre used by the reduction.  Returns the count. */
int ophys_probe_ball_contacts(const OWorld* w, const float* center, int* tri, float* point, float* normal,
                              float* depth, float* reduction)
{
    OBallContact cs[MAX_BALL_CONTACTS];
    const int n = gather_ball_contacts(w->arena, v3(center[0], center[1], center[2]), cs);
    for (int i = 0; i < n; i++) {
        tri[i] = cs[i].tri;
        point[3 * i] = cs[i].point.x; point[3 * i + 1] = cs[i].point.y; point[3 * i + 2] = cs[i].point.z;
        normal[3 * i] = cs[i].normal.x; normal[3 * i + 1] = cs[i].normal.y; normal[3 * i + 2] = cs[i].normal.z;
        depth[i] = cs[i].depth;
        reduction[3 * i] = cs[i].reductionPos.x; reduction[3 * i + 1] = cs[i].reductionPos.y;
        reduction[3 * i + 2] = cs[i].reductionPos.z;
    }
    return n;
}

int ophys_ball_hit_prev_tick(int hitTick, int tick) { return hitTick >= 0 && tick > 0 && hitTick == tick - 1; }

/* ------------------------------------------------------------- ball vs car */

typedef struct { V3 pos, cen, vel, ang; Q4 rot; } OBCBody;
typedef struct { V3 axis, ballTorque, carAngular; float jacInv, applied; } OBCRow;

static OBCRow bc_row(const OBCBody* car, V3 axis, V3 ballOff, V3 carOff)
{
    OBCRow r;
    memset(&r, 0, sizeof r);
    r.axis = axis;
    r.ballTorque = vcross(ballOff, axis);
    const V3 ct = vcross(carOff, axis);
    r.carAngular = qworld(car->rot, vmul(qlocal(car->rot, ct), K_CAR_INV_INERTIA));
    const float denom = K_BALL_INV_MASS + K_CAR_INV_MASS + K_BALL_INV_INERTIA * vlensq(r.ballTorque) + vdot(r.carAngular, ct);
    r.jacInv = 1.f / o_max(denom, 1e-8f);
    return r;
}

static float bc_vel(const OBCRow* r, V3 bv, V3 ba, const OBCBody* car, V3 ballOff, V3 carOff)
{
    const V3 bp = vadd(bv, vcross(ba, ballOff));
    const V3 cp = vadd(car->vel, vcross(car->ang, carOff));
    return vdot(r->axis, vsub(bp, cp));
}

static void bc_apply(V3* bv, V3* ba, OBCBody* car, const OBCRow* r, float imp)
{
    *bv = vadd(*bv, vscale(r->axis, imp * K_BALL_INV_MASS));
    *ba = vadd(*ba, vscale(r->ballTorque, imp * K_BALL_INV_INERTIA));
    car->vel = vsub(car->vel, vscale(r->axis, imp * K_CAR_INV_MASS));
    car->ang = vsub(car->ang, vscale(r->carAngular, imp));
}

static float extra_curve(float s)
{
    if (s <= 500.f) return 0.65f;
    if (s <= 2300.f) return 0.65f + (0.55f - 0.65f) * ((s - 500.f) / 1800.f);
    if (s <= 4600.f) return 0.55f + (0.30f - 0.55f) * ((s - 2300.f) / 2300.f);
    return 0.30f;
}

/* include/Physics/CarBall/Solve.cuh:207-243 */
static void ball_car_pair(OWorld* w, int sim, int ci, V3 preSolveBallVel)
{
    OSim* s = &w->sims[sim];
    OCar* c = &w->cars[ci];
    if (c->demoed) return;
    const V3 ballPos = s->pos;
    V3 ballVel = s->vel, ballAng = s->ang;
    OBCBody car = { c->pos, c->cen, c->vel, c->ang, c->rot };
    const V3 preCarVel = car.vel;

    /* sphereOBBContact (include/Physics/CarBall/Contact.cuh:13-77) */
    const V3 CORE = v3(K_CAR_HALF.x - K_CARBALL_MARGIN, K_CAR_HALF.y - K_CARBALL_MARGIN, K_CAR_HALF.z - K_CARBALL_MARGIN);
    const V3 lb = qlocal(car.rot, vsub(ballPos, car.cen));
    const V3 cl = v3(o_clamp(lb.x, -CORE.x, CORE.x), o_clamp(lb.y, -CORE.y, CORE.y), o_clamp(lb.z, -CORE.z, CORE.z));
    const V3 dl = vsub(lb, cl);
    const float dsq = vlensq(dl);
    const float inter = K_BALL_RADIUS + K_CARBALL_MARGIN;
    const float accept = inter + K_CARBALL_BREAK;
    V3 point, normal;
    float depth;
    if (dsq > 1e-8f) {
        if (dsq >= accept * accept) return;
        const float dist = sqrtf(dsq);
        const V3 ln = vscale(dl, 1.f / dist);
        point = vadd(car.cen, qworld(car.rot, vadd(cl, vscale(ln, K_CARBALL_MARGIN))));
        normal = qworld(car.rot, ln);
        depth = inter - dist;
    } else {
        const V3 fd = vsub(CORE, vabs(lb));
        int axis = 0;
        float md = fd.x;
        if (fd.y < md) { axis = 1; md = fd.y; }
        if (fd.z < md) { axis = 2; md = fd.z; }
        V3 ln = V_ZERO;
        vset(&ln, axis, vget(lb, axis) >= 0.f ? 1.f : -1.f);
        point = vadd(car.cen, qworld(car.rot, vadd(cl, vscale(ln, K_CARBALL_MARGIN))));
        normal = qworld(car.rot, ln);
        depth = inter + md;
    }

    /* makeBallCarConstraint */
    const V3 ballOff = vscale(normal, -K_BALL_RADIUS);
    const V3 carOff = vsub(point, car.pos);
    OBCRow nr = bc_row(&car, normal, ballOff, carOff);
    const float relN = bc_vel(&nr, ballVel, ballAng, &car, ballOff, carOff);
    V3 tan = vsub(vadd(ballVel, vcross(ballAng, ballOff)), vadd(car.vel, vcross(car.ang, carOff)));
    tan = vsub(tan, vscale(normal, relN));
    const float tl = vlensq(tan);
    const float restitution = fabsf(relN) > K_RESTITUTION_VEL_THRESH ? K_CARBALL_RESTITUTION * -relN : 0.f;
    tan = tl > K_FLT_EPS ? vscale(tan, o_rsqrt(tl)) : fallback_tangent(normal);
    OBCRow fr = bc_row(&car, tan, ballOff, carOff);

    for (int it = 0; it < K_SOLVER_ITERS; it++) {
        const float rn = bc_vel(&nr, ballVel, ballAng, &car, ballOff, carOff);
        const float ni = solve_lower(restitution * nr.jacInv, 0.f, nr.jacInv, rn, 0.f, &nr.applied);
        bc_apply(&ballVel, &ballAng, &car, &nr, ni);
        const float rt = bc_vel(&fr, ballVel, ballAng, &car, ballOff, carOff);
        const float maxF = K_CARBALL_FRICTION * nr.applied;
        const float fi = solve_impulse(0.f, 0.f, fr.jacInv, rt, -maxF, maxF, &fr.applied);
        bc_apply(&ballVel, &ballAng, &car, &fr, fi);
    }
    s->vel = ballVel; s->ang = ballAng;
    c->vel = car.vel; c->ang = car.ang;

    /* applyBallCarSplitCorrection */
    const float pen = depth - K_LINEAR_SLOP;
    if (pen > 0.f) {
        const float push = pen * K_CONTACT_ERP / K_DT * nr.jacInv;
        const V3 ballCorr = vscale(normal, push * K_BALL_INV_MASS * K_DT);
        const V3 carCorr = vscale(normal, -push * K_CAR_INV_MASS * K_DT);
        const V3 turn = vscale(nr.carAngular, -push);
        s->pos = vadd(s->pos, ballCorr);
        const V3 cp = vadd(c->pos, carCorr);
        c->pos = cp;
        const Q4 cr = ophys_integrate_quat(c->rot, vscale(turn, K_SPLIT_TURN_ERP));
        c->rot = cr;
        c->cen = vadd(cp, qworld(cr, K_CAR_OFFSETS));
    }

    /* applyBallCarExtraImpulse (include/Physics/CarBall/ExtraImpulse.cuh:58-79) */
    const int tick = w->tickCount;
    c->ballContactTick = tick;
    s->lastTouch = tick;
    const int last = c->ballHitTick;
    if (tick <= last + 1 && last <= tick) return;
    c->ballHitTick = tick;
    const V3 relVel = vsub(preSolveBallVel, preCarVel);
    const float raw = sqrtf(vlensq(relVel));
    const float speed = o_min(raw, K_EXTRA_MAXDV);
    V3 added = V_ZERO;
    if (speed > 0.f) {
        const V3 rp = vsub(ballPos, car.pos);
        V3 hd = v3(rp.x, rp.y, rp.z * K_EXTRA_Z_SCALE);
        const float hl = vlensq(hd);
        if (hl > 1e-12f) {
            hd = vscale(hd, o_rsqrt(hl));
            const V3 fwd = qworld(car.rot, V_X);
            const float fs = vdot(hd, fwd) * (1.f - K_EXTRA_FWD_SCALE);
            hd = vsub(hd, vscale(fwd, fs));
            const float al = vlensq(hd);
            if (al > 1e-12f) hd = vscale(hd, o_rsqrt(al));
            added = vscale(hd, speed * extra_curve(speed));
        }
    }
    s->imp = vadd(s->imp, added);
}

/* include/Physics/BallArena/Solve.cuh:56-117 */
static void solve_ball(OWorld* w, int sim)
{
    OSim* s = &w->sims[sim];
    const V3 ballVel = s->vel, ballAng = s->ang;
    const int sleeping = vlensq(ballVel) == 0.f && vlensq(ballAng) == 0.f;
    const V3 exported = s->pos;
    const int valid = s->intValid != 0;
    V3 posBT = valid && vlensq(vsub(exported, s->expPos)) == 0.f ? s->intPos : vscale(exported, .02f);
    V3 velBT = valid && vlensq(vsub(ballVel, s->expVel)) == 0.f ? s->intVel : vscale(ballVel, .02f);
    const V3 damped = sleeping ? velBT : vscale(velBT, K_BALL_DRAG_FACTOR);
    const V3 preBT = sleeping ? velBT : vadd(damped, vscale(vscale(K_GRAVITY, .02f), K_DT));
    const V3 velNoExt = vscale(damped, 50.f);
    const V3 preVel = vscale(preBT, 50.f);
    V3 pushVel = V_ZERO;
    if (!sleeping) {
        OBallBody b;
        memset(&b, 0, sizeof b);
        b.pos = s->pos; b.vel = preVel; b.velNoExt = velNoExt; b.ang = s->ang;
        OBallContact cs[MAX_BALL_CONTACTS];
        const int count = gather_ball_contacts(w->arena, b.pos, cs);
        int hit = 0;
        for (int k = 0; k < w->nCars; k++)
            hit |= ophys_ball_hit_prev_tick(w->cars[sim * w->nCars + k].ballHitTick, w->tickCount);
        solve_ball_contacts(&b, cs, count, hit);
        s->vel = b.vel; s->ang = b.ang;
        pushVel = b.pushVel;
    }

    /* solveBallCarForSim (include/Physics/CarBall/Solve.cuh:245-265) */
    {
        const V3 bp = s->pos;
        const V3 SOLVER_HALF = v3(K_CAR_HALF.x + K_CARBALL_MARGIN, K_CAR_HALF.y + K_CARBALL_MARGIN, K_CAR_HALF.z + K_CARBALL_MARGIN);
        const float maxDist = K_BALL_RADIUS + vlen(SOLVER_HALF);
        for (int k = 0; k < w->nCars; k++) {
            const int ci = sim * w->nCars + k;
            if (w->cars[ci].demoed) continue;
            if (vlensq(vsub(bp, w->cars[ci].cen)) > maxDist * maxDist) continue;
            ball_car_pair(w, sim, ci, preVel);
        }
    }

    const V3 corrected = s->pos;
    if (vlensq(vsub(corrected, exported)) != 0.f) posBT = vscale(corrected, .02f);
    const V3 finalVel = s->vel;
    velBT = vlensq(vsub(finalVel, preVel)) == 0.f ? preBT : vscale(finalVel, .02f);
    posBT = vadd(posBT, vscale(vscale(pushVel, .02f), K_DT));
    posBT = vadd(posBT, vscale(velBT, K_DT));
    const V3 ballPos = vscale(posBT, 50.f);
    s->pos = ballPos;
    s->intPos = posBT; s->intVel = velBT;
    s->expPos = ballPos; s->expVel = finalVel;
    s->intValid = 1;

    /* detectGoal (include/Physics/Goals.cuh:6-32) */
    const float thr = K_GOAL_THRESHOLD_Y + K_BALL_RADIUS;
    const int scorer = ballPos.y > thr ? 1 : (ballPos.y < -thr ? -1 : 0);
    if (!scorer || s->lastScorer != 0) return;
    if (scorer > 0) s->blue++; else s->orange++;
    s->lastScorer = scorer;
    s->goalTick = w->tickCount;
}

/* ------------------------------------------------------------ finish, pads */

static void respawn_car(OWorld* w, int ci)
{
    OCar* c = &w->cars[ci];
    const int local = ci % w->nCars;
    const OSpawn sp = respawn_loc(c->in.respawnIdx);
    const int orange = local >= w->nBlue;
    const float y = orange ? -sp.y : sp.y;
    const float yaw = orange ? sp.yaw + K_PI : sp.yaw;
    const Q4 rot = qangle(yaw);
    c->pos = v3(sp.x, y, K_CAR_RESPAWN_Z);
    c->cen = vadd(c->pos, qworld(rot, K_CAR_OFFSETS));
    c->rot = rot;
    c->vel = V_ZERO; c->ang = V_ZERO; c->imp = V_ZERO;
    c->demoed = 0; c->demoTimer = 0.f; c->contactIdx = -1; c->contactCooldown = 0.f;
    c->ballHitTick = -1; c->ballContactTick = -1;
    for (int k = 0; k < N_WHEELS; k++) c->wheelContact[k] = 0;
    memset(&c->in, 0, sizeof c->in);
    c->in.onGround = 1;
    c->in.boost = K_BOOST_SPAWN;
}

/* include/Physics/FinishTick.cuh:100-141 */
static void finish_car(OWorld* w, int ci)
{
    OCar* c = &w->cars[ci];
    if (c->demoed) {
        float timer = c->demoTimer;
        if (timer <= K_DEMO_RESPAWN_TIME) {
            const float st = c->ctrl.steer;
            const int dir = st < -K_DEMO_INPUT_DEADZONE ? -1 : (st > K_DEMO_INPUT_DEADZONE ? 1 : 0);
            if (dir != 0 && dir != c->in.lastRespawnDir) {
                if (dir < 0 && c->in.respawnIdx > 0) c->in.respawnIdx--;
                else if (dir > 0 && c->in.respawnIdx < 3) c->in.respawnIdx++;
            }
            c->in.lastRespawnDir = dir;
        }
        timer = o_max(timer - K_DT, 0.f);
        c->demoTimer = timer;
        if (timer <= 0.f) respawn_car(w, ci);
        return;
    }
    const V3 imp = c->imp;
    if (vlensq(imp) > 1e-12f) {
        V3 vel = vadd(c->vel, imp);
        const float ss = vlensq(vel);
        if (ss > K_CAR_MAX_SPEED * K_CAR_MAX_SPEED) vel = vscale(vel, K_CAR_MAX_SPEED * o_rsqrt(ss));
        c->vel = vel;
        c->imp = V_ZERO;
    }
    float cd = c->contactCooldown;
    if (cd <= 0.f) return;
    c->contactCooldown = o_max(cd - K_DT, 0.f);
}

static void finish_ball(OSim* s)
{
    V3 vel = vadd(s->vel, s->imp);
    V3 ang = s->ang;
    float ss = vlensq(vel);
    if (ss > K_BALL_MAX_SPEED * K_BALL_MAX_SPEED) vel = vscale(vel, K_BALL_MAX_SPEED * o_rsqrt(ss));
    ss = vlensq(ang);
    if (ss > K_BALL_MAX_ANG * K_BALL_MAX_ANG) ang = vscale(ang, K_BALL_MAX_ANG * o_rsqrt(ss));
    s->vel = vel; s->ang = ang; s->imp = V_ZERO;
}

/* include/Physics/BoostPads.cuh:58-106 */
static void boost_pads(OWorld* w, int sim)
{
    OSim* s = &w->sims[sim];
    for (int p = 0; p < N_PADS; p++) {
        float cd = s->pads[p];
        if (cd > 0.f) { cd = o_max(cd - K_DT, 0.f); s->pads[p] = cd; }
        if (cd > 0.f) continue;
        const int big = p < 6;
        const float radius = big ? K_BIG_PAD_RADIUS : K_SMALL_PAD_RADIUS;
        const V3 pp = ophys_pad_pos(p);
        int locked = -1;
        for (int k = 0; k < w->nCars; k++) {
            const int ci = sim * w->nCars + k;
            if (w->cars[ci].demoed) continue;
            const V3 cp = w->cars[ci].pos;
            const float dx = cp.x - pp.x, dy = cp.y - pp.y;
            const float dsq = dx * dx + dy * dy;
            if (dsq < radius * radius && fabsf(cp.z - pp.z) < K_PAD_HEIGHT) locked = ci;
        }
        if (locked < 0) continue;
        OInternal* in = &w->cars[locked].in;
        if (in->boost >= K_BOOST_MAX) continue;
        in->boost = o_min(in->boost + (big ? K_BIG_PAD_AMOUNT : K_SMALL_PAD_AMOUNT), K_BOOST_MAX);
        s->pads[p] = big ? K_BIG_PAD_COOLDOWN : K_SMALL_PAD_COOLDOWN;
    }
}

/* ---------------------------------------------------------------- the tick */

void ophys_tick(OWorld* w, int kind, const void* actions)
{
    /* beginStep */
    w->tickCount++;
    for (int s = 0; s < w->nSim; s++) w->sims[s].episodeTicks++;
    /* broad + suspension raycast */
    for (int c = 0; c < w->nTotal; c++) ophys_broadphase(w, c);
    for (int c = 0; c < w->nTotal; c++) ophys_raycast(w, c);
    /* controls */
    for (int c = 0; c < w->nTotal; c++) {
        ophys_controls_decode(kind, actions, c, &w->cars[c].ctrl);
        process_controls(w, &w->cars[c]);
    }
    /* narrow phase */
    for (int c = 0; c < w->nTotal; c++) car_arena_sat(w, c);
    for (int c = 0; c < w->nTotal; c++) car_arena_clip(w, c);
    /* manifold + solve */
    for (int c = 0; c < w->nTotal; c++) solve_car_arena(w, c);
    /* car-car + ball */
    for (int s = 0; s < w->nSim; s++) {
        const int base = s * w->nCars;
        for (int a = 0; a < w->nCars - 1; a++)
            for (int b = a + 1; b < w->nCars; b++) car_car_pair(w, base + b, base + a);
        solve_ball(w, s);
    }
    /* integrate cars */
    for (int c = 0; c < w->nTotal; c++) {
        OCar* car = &w->cars[c];
        if (car->demoed) continue;
        OBody b = load_body(car);
        integrate_state(&b.pos, &b.cen, &b.rot, b.vel, b.ang);
        clamp_body(&b);
        store_body(car, &b);
    }
    /* impulse cache */
    for (int s = 0; s < w->nSim; s++) finish_ball(&w->sims[s]);
    for (int c = 0; c < w->nTotal; c++) finish_car(w, c);
    /* boost pads */
    for (int s = 0; s < w->nSim; s++) boost_pads(w, s);
}

/* ----------------------------------------------------------------- resets */

static void reset_car_kickoff(OWorld* w, int ci, int loc, int invert)
{
    OCar* c = &w->cars[ci];
    const OSpawn sp = kickoff_loc(loc % 5);
    const float x = invert ? -sp.x : sp.x;
    const float y = invert ? -sp.y : sp.y;
    const float yaw = invert ? sp.yaw + K_PI : sp.yaw;
    c->pos = v3(x, y, sp.z);
    c->vel = V_ZERO; c->ang = V_ZERO;
    c->rot = qangle(yaw);
    c->cen = vadd(c->pos, qworld(c->rot, K_CAR_OFFSETS));
    c->imp = V_ZERO;
    c->demoed = 0; c->demoTimer = 0.f; c->contactIdx = -1; c->contactCooldown = 0.f;
    c->ballHitTick = -1; c->ballContactTick = -1;
    memset(&c->ctrl, 0, sizeof c->ctrl);
    for (int k = 0; k < N_WHEELS; k++) c->wheelContact[k] = 0;
    memset(&c->in, 0, sizeof c->in);
    c->in.onGround = 1;
    c->in.boost = K_BOOST_SPAWN;
}

/* include/State/Reset.cuh:51-80 */
void ophys_reset_to_kickoff(OWorld* w, int sim)
{
    const uint32_t seed = o_hash32((uint32_t)w->seed) ^ o_hash32((uint32_t)sim) ^ o_hash32((uint32_t)w->tickCount);
    const int perm = o_random_index(seed, 120);
    OSim* s = &w->sims[sim];
    s->pos = v3(0.f, 0.f, K_BALL_REST_Z);
    s->vel = V_ZERO; s->ang = V_ZERO;
    s->intValid = 0;
    for (int team = 0; team < 2; team++) {
        const int size = team ? w->nOrange : w->nBlue;
        for (int i = 0; i < size; i++) {
            const int ci = sim * w->nCars + (team * w->nBlue + i);
            reset_car_kickoff(w, ci, ophys_kickoff_perm(perm, i), team);
        }
    }
}

/* GameState::reset + Workspace::reset + resetKernel (GameState.cuh:221-231,
 * Workspace.cuh:225-233, Kernels.cu:15-23). */
void ophys_reset_all(OWorld* w)
{
    w->tickCount = 0;
    for (int s = 0; s < w->nSim; s++) {
        OSim* sm = &w->sims[s];
        sm->episodeTicks = 0;
        sm->lastTouch = 0;
        sm->imp = V_ZERO;
        sm->intValid = 0;
        for (int p = 0; p < N_PADS; p++) sm->pads[p] = 0.f;
        sm->blue = sm->orange = sm->lastScorer = sm->goalTick = sm->overtime = 0;
        sm->ballArenaContactTick = -1;
    }
    for (int ci = 0; ci < w->nTotal; ci++) {
        OCar* c = &w->cars[ci];
        c->imp = V_ZERO;
        c->demoed = 0; c->demoTimer = 0.f;
        c->contactIdx = -1; c->contactCooldown = 0.f;
        c->ballHitTick = -1; c->ballContactTick = -1;
        for (int k = 0; k < N_WHEELS; k++) { c->wheelSource[k] = SRC_NONE; c->wheelContact[k] = 0; }
        c->arenaContactTick = -1;
        memset(&c->in, 0, sizeof c->in);
        c->in.onGround = 1;
        c->in.boost = K_BOOST_SPAWN;
        c->numTris = 0; c->hitCount = 0; c->manCount = 0;
        for (int k = 0; k < N_WHEELS; k++) { c->latF[k] = 0.f; c->lonF[k] = 0.f; }
        c->brake = c->brakePrev = c->throttleVal = c->rawThrottle = c->handbrakeVal = 0.f;
        c->steer = c->steerPrev = c->drive = c->drivePrev = 0.f;
        c->jumpImp = V_ZERO; c->angImp = V_ZERO;
    }
    for (int s = 0; s < w->nSim; s++) ophys_reset_to_kickoff(w, s);
}

/* include/State/Reset.cuh:82-171 */
void ophys_reset_after_done(OWorld* w, int sim, int maxTicks, int overtimeTicks, int noTouchTicks)
{
    OSim* s = &w->sims[sim];
    const int scored = s->lastScorer != 0;
    const int sinceTouch = w->tickCount - s->lastTouch;
    const int noTouch = noTouchTicks > 0 && sinceTouch >= noTouchTicks;
    const int otExpired = s->overtime && s->episodeTicks >= maxTicks + overtimeTicks;
    const int timeout = s->episodeTicks >= maxTicks;
    if (!s->overtime && !scored && !noTouch && s->episodeTicks >= maxTicks && s->blue == s->orange) {
        s->overtime = 1;
        return;
    }
    if (!(scored || noTouch || otExpired || (!s->overtime && timeout))) return;
    s->blue = s->orange = s->lastScorer = s->goalTick = s->overtime = 0;
    ophys_reset_to_kickoff(w, sim);
    s->episodeTicks = 0;
    s->lastTouch = w->tickCount;
    s->ballArenaContactTick = -1;
    for (int k = 0; k < w->nCars; k++) {
        OCar* c = &w->cars[sim * w->nCars + k];
        c->arenaContactTick = -1;
        c->numTris = 0; c->hitCount = 0; c->manCount = 0;
        c->brake = c->brakePrev = c->throttleVal = c->rawThrottle = c->handbrakeVal = 0.f;
        c->steer = c->steerPrev = c->drive = c->drivePrev = 0.f;
        c->jumpImp = V_ZERO; c->angImp = V_ZERO;
        for (int q = 0; q < N_WHEELS; q++) {
            c->wheelSource[q] = SRC_NONE; c->wheelContact[q] = 0;
            c->rayDist[q] = 0.f; c->rayNormal[q] = V_ZERO;
            c->latF[q] = 0.f; c->lonF[q] = 0.f;
        }
    }
    for (int p = 0; p < N_PADS; p++) s->pads[p] = 0.f;
}

/* ------------------------------------------------------------------ probes */

static OWorld* probe_world(void)
{
    static OWorld w;
    static OCar cars[2];
    static OSim sims[1];
    memset(&w, 0, sizeof w);
    memset(cars, 0, sizeof cars);
    memset(sims, 0, sizeof sims);
    w.nSim = 1; w.nBlue = 1; w.nOrange = 1; w.nCars = 2; w.nTotal = 2; w.seed = 42;
    w.cars = cars; w.sims = sims;
    return &w;
}

/* tests/physics_regressions.cu:38-76: tryStartDodge on an identity-oriented car */
void ophys_probe_dodge(float pitch, float yaw, float roll, int* hasFlipped, int* hasDoubleJumped, float* vel)
{
    OWorld* w = probe_world();
    OCar* c = &w->cars[0];
    c->ctrl.pitch = pitch; c->ctrl.yaw = yaw; c->ctrl.roll = roll;
    OCtx x;
    memset(&x, 0, sizeof x);
    x.w = w; x.c = c;
    x.rot = qangle(0.f);
    x.fwd = V_X; x.up = V_Z;
    x.jumpPressed = 1;
    try_start_dodge(&x);
    *hasFlipped = c->in.hasFlipped;
    *hasDoubleJumped = c->in.hasDoubleJumped;
    vel[0] = c->vel.x; vel[1] = c->vel.y; vel[2] = c->vel.z;
}

/* tests/turtle_recovery.cu:5-16: updateAutoFlip with a given previous manifold */
void ophys_probe_autoflip(const float* quat, int jump, int contacts, const float* normal,
                          int* isAutoFlipping, float* timer, float* ang)
{
    OWorld* w = probe_world();
    OCar* c = &w->cars[0];
    c->manCount = contacts;
    c->manNormal = v3(normal[0], normal[1], normal[2]);
    OCtx x;
    memset(&x, 0, sizeof x);
    x.w = w; x.c = c;
    x.rot = q4(quat[0], quat[1], quat[2], quat[3]);
    x.fwd = qworld(x.rot, V_X);
    x.up = qworld(x.rot, V_Z);
    x.jumpPressed = jump;
    update_autoflip(&x);
    *isAutoFlipping = c->in.isAutoFlipping;
    *timer = c->in.autoFlipTimer;
    ang[0] = c->ang.x; ang[1] = c->ang.y; ang[2] = c->ang.z;
}

/* tests/physics_regressions.cu:25-36: one floor contact, split correction */
float ophys_probe_ball_floor_split(float depth, float velz, int ballWasHit)
{
    OBallBody b;
    memset(&b, 0, sizeof b);
    b.vel = v3(0.f, 0.f, velz);
    b.velNoExt = b.vel;
    OBallContact ct;
    memset(&ct, 0, sizeof ct);
    ct.normal = V_Z;
    ct.relPos = v3(0.f, 0.f, -K_BALL_RADIUS);
    ct.depth = depth;
    solve_ball_contacts(&b, &ct, 1, ballWasHit);
    return b.pushVel.z;
}

/* tests/physics_regressions.cu:104-112: steer staging lag */
void ophys_probe_steer_stage(float staged, float* prevOut, float* curOut)
{
    OWorld* w = probe_world();
    OCar* c = &w->cars[0];
    c->steer = staged;
    OCtx x;
    memset(&x, 0, sizeof x);
    x.w = w; x.c = c;
    update_steer(&x);
    *prevOut = c->steerPrev;
    *curOut = c->steer;
}

/* box-triangle SAT of a triangle given in box-local coordinates (SAT.cuh:42-121) */
void ophys_probe_box_tri_sat(const float* tri, int* overlap, int* axisIdx, float* depth, float* axis)
{
    OTri t;
    tri_set(&t, v3(tri[0], tri[1], tri[2]), v3(tri[3], tri[4], tri[5]), v3(tri[6], tri[7], tri[8]));
    t.delta = vneg(tri_center(&t));
    const OSat s = tri_sat(&t);
    *overlap = s.overlap;
    *axisIdx = s.axisIdx;
    *depth = s.minPen;
    axis[0] = s.minAxis.x; axis[1] = s.minAxis.y; axis[2] = s.minAxis.z;
}

/* The arena manifold of car ci built from the current state: broadphase,
 * SAT, clip, then the plane points and the best mesh contact
 * (include/Physics/CarArena/Manifold.cuh:198-310) */
int ophys_probe_manifold(OWorld* w, int ci, float* carPos, float* worldPos, float* normal, float* dist)
{
    ophys_broadphase(w, ci);
    car_arena_sat(w, ci);
    car_arena_clip(w, ci);
    OManPoint pts[MAX_MANIFOLD];
    const int n = build_manifold(w, ci, pts);
    for (int i = 0; i < n; i++) {
        const float* src[3] = { &pts[i].carPos.x, &pts[i].worldPos.x, &pts[i].worldNormal.x };
        float* dst[3] = { carPos + 3 * i, worldPos + 3 * i, normal + 3 * i };
        for (int k = 0; k < 3; k++) { dst[k][0] = src[k][0]; dst[k][1] = src[k][1]; dst[k][2] = src[k][2]; }
        dist[i] = pts[i].dist;
    }
    return n;
}

/* SAT and clip contacts of one triangle given in box-local coordinates,
 * as the car-arena stages generate them (no internal-edge adjustment) */
int ophys_probe_box_tri_contacts(const float* tri, int* axisIdx, float* carPos, float* arenaPos, float* normal,
                                 float* depth)
{
    OTriClip tc;
    tri_set(&tc.t, v3(tri[0], tri[1], tri[2]), v3(tri[3], tri[4], tri[5]), v3(tri[6], tri[7], tri[8]));
    tc.t.delta = vneg(tri_center(&tc.t));
    tc.faceNormal = vnorm(vcross(tc.t.e0, vsub(tc.t.v2, tc.t.v0)));
    tc.angles = v3(K_BOUNDARY_EDGE_ANGLE, K_BOUNDARY_EDGE_ANGLE, K_BOUNDARY_EDGE_ANGLE);
    const OSat s = tri_sat(&tc.t);
    *axisIdx = s.overlap ? s.axisIdx : -1;
    if (!s.overlap) return 0;
    OContact ct[MAX_PAIR_CONTACTS];
    const int n = clip_pair(&tc, s.axisIdx, s.minPen, s.minAxis, ct);
    for (int i = 0; i < n; i++) {
        const float* src[3] = { &ct[i].carPos.x, &ct[i].arenaPos.x, &ct[i].normal.x };
        float* dst[3] = { carPos + 3 * i, arenaPos + 3 * i, normal + 3 * i };
        for (int k = 0; k < 3; k++) { dst[k][0] = src[k][0]; dst[k][1] = src[k][1]; dst[k][2] = src[k][2]; }
        depth[i] = ct[i].depth;
    }
    return n;
}

/* SAT and contacts of two car hitboxes given in world coordinates, as the
 * car-car stage generates them; points in each box's local frame */
int ophys_probe_box_box_contacts(const float* cenA, const float* rotA, const float* cenB, const float* rotB,
                                 int* axisIdx, float* carPosA, float* carPosB, float* normal, float* depth)
{
    const OBox A = { v3(cenA[0], cenA[1], cenA[2]), q4(rotA[0], rotA[1], rotA[2], rotA[3]) };
    const OBox B = { v3(cenB[0], cenB[1], cenB[2]), q4(rotB[0], rotB[1], rotB[2], rotB[3]) };
    const OSat s = cc_sat(&A, &B);
    *axisIdx = s.overlap ? s.axisIdx : -1;
    if (!s.overlap) return 0;
    OCC cts[MAX_MANIFOLD];
    const int n = cc_contacts(&s, &A, &B, cts);
    for (int i = 0; i < n; i++) {
        const float* src[3] = { &cts[i].carPosA.x, &cts[i].carPosB.x, &cts[i].normal.x };
        float* dst[3] = { carPosA + 3 * i, carPosB + 3 * i, normal + 3 * i };
        for (int k = 0; k < 3; k++) { dst[k][0] = src[k][0]; dst[k][1] = src[k][1]; dst[k][2] = src[k][2]; }
        depth[i] = cts[i].depth;
    }
    return n;
}

/* box-box SAT of two car hitboxes (CarCar/SAT.cuh:46-125) */
void ophys_probe_box_box_sat(const float* cenA, const float* rotA, const float* cenB, const float* rotB,
                             int* overlap, int* axisIdx, float* depth)
{
    const OBox A = { v3(cenA[0], cenA[1], cenA[2]), q4(rotA[0], rotA[1], rotA[2], rotA[3]) };
    const OBox B = { v3(cenB[0], cenB[1], cenB[2]), q4(rotB[0], rotB[1], rotB[2], rotB[3]) };
    const OSat s = cc_sat(&A, &B);
    *overlap = s.overlap;
    *axisIdx = s.axisIdx;
    *depth = s.minPen;
}
