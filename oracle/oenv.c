/*
 * oenv.c - environment layer of the CPU oracle: output buffers, packing,
 * setters, checkpoint export/import and the multi-threaded CPU run.
 *
 * TEST INFRASTRUCTURE (see omath.h).  Restates
 *   EnvWrapper sequencing          python/carl.cu:286-706
 *   packing kernels                src/EnvIO.cu:47-357, 603-643
 *   observation / state / rewards  include/Physics/Observations.cuh:9-397
 *   layout contract                include/Cuda/DLPack.h:60-107
 */
#define _POSIX_C_SOURCE 200809L
#include <pthread.h>
#include <stdlib.h>
#include <string.h>
#include <time.h>

#include "../include/carl_amd.h"
#include "carl_oracle.h"
#include "ointernal.h"

#define OBS_PER_CAR 21
#define STATE_PER_CAR 22

struct OEnv {
    OWorld w;
    int frameskip, invert, normalize, prevControls;
    int maxTicks, overtimeTicks, noTouchTicks;
    int obsDim, stateDim;
    float *obs, *tobs, *state, *tstate, *rewards;
    uint8_t *dones, *overtime, *tovertime;
    int32_t *score, *ticks, *tscore, *tticks;
    int32_t* actions;
    float* cactions;
};

static int obs_dim(int nCars, int prev)
{
    return 9 + nCars * OBS_PER_CAR + 2 * N_PADS + 6 + (nCars - 1) * 6 + 6 + 2 + 5 + (prev ? 8 : 0);
}

/* ------------------------------------------------------------------ packing */

static V3 obs_vec(V3 v, int inv) { return inv ? v3(-v.x, -v.y, v.z) : v; }

static const int INVERTED_PAD[N_PADS] = {
    1, 0, 5, 4, 3, 2, 33, 32, 31, 30, 29, 28, 27, 26, 25, 24, 23,
    22, 21, 20, 19, 18, 17, 16, 15, 14, 13, 12, 11, 10, 9, 8, 7, 6
};

static void put3(float* o, int* k, V3 v) { o[(*k)++] = v.x; o[(*k)++] = v.y; o[(*k)++] = v.z; }

static void pack_car(const OWorld* w, int ci, int inv, float* o, int* k)
{
    const OCar* c = &w->cars[ci];
    put3(o, k, obs_vec(c->pos, inv));
    put3(o, k, obs_vec(c->vel, inv));
    put3(o, k, obs_vec(c->ang, inv));
    put3(o, k, obs_vec(qworld(c->rot, V_X), inv));
    put3(o, k, obs_vec(qworld(c->rot, V_Z), inv));
    o[(*k)++] = c->in.boost;
    o[(*k)++] = (float)c->in.onGround;
    o[(*k)++] = (float)(c->demoed != 0);
    o[(*k)++] = (float)c->in.hasFlipped;
    o[(*k)++] = (float)c->in.hasDoubleJumped;
    o[(*k)++] = (float)c->in.isBoosting;
}

/* include/Physics/Observations.cuh:97-238 */
static void pack_observation(const OEnv* e, int sim, int obsIdx, float* o)
{
    const OWorld* w = &e->w;
    const int nC = w->nCars, base = sim * nC;
    const int orange = obsIdx >= w->nBlue;
    const int inv = e->invert && orange;
    int k = 0;
    const OSim* s = &w->sims[sim];
    const V3 egoPos = w->cars[base + obsIdx].pos, egoVel = w->cars[base + obsIdx].vel;
    put3(o, &k, obs_vec(s->pos, inv));
    put3(o, &k, obs_vec(s->vel, inv));
    put3(o, &k, obs_vec(s->ang, inv));
    pack_car(w, base + obsIdx, inv, o, &k);
    const int tS = orange ? w->nBlue : 0, tE = orange ? nC : w->nBlue;
    for (int c = tS; c < tE; c++) if (c != obsIdx) pack_car(w, base + c, inv, o, &k);
    const int oS = orange ? 0 : w->nBlue, oE = orange ? w->nBlue : nC;
    for (int c = oS; c < oE; c++) pack_car(w, base + c, inv, o, &k);
    for (int p = 0; p < N_PADS; p++) {
        const int pi = inv ? INVERTED_PAD[p] : p;
        o[k++] = s->pads[pi] <= 0.f;
    }
    for (int p = 0; p < N_PADS; p++) {
        const int pi = inv ? INVERTED_PAD[p] : p;
        o[k++] = vlen(vsub(egoPos, ophys_pad_pos(pi)));
    }
    put3(o, &k, obs_vec(vsub(s->pos, egoPos), inv));
    put3(o, &k, obs_vec(vsub(s->vel, egoVel), inv));
    for (int c = tS; c < tE; c++) {
        if (c == obsIdx) continue;
        put3(o, &k, obs_vec(vsub(w->cars[base + c].pos, egoPos), inv));
        put3(o, &k, obs_vec(vsub(w->cars[base + c].vel, egoVel), inv));
    }
    for (int c = oS; c < oE; c++) {
        put3(o, &k, obs_vec(vsub(w->cars[base + c].pos, egoPos), inv));
        put3(o, &k, obs_vec(vsub(w->cars[base + c].vel, egoVel), inv));
    }
    const float ownY = orange ? K_GOAL_CENTER_Y : -K_GOAL_CENTER_Y;
    const V3 own = v3(0.f, ownY, K_GOAL_CENTER_Z), opp = v3(0.f, -ownY, K_GOAL_CENTER_Z);
    put3(o, &k, obs_vec(vsub(own, s->pos), inv));
    put3(o, &k, obs_vec(vsub(opp, s->pos), inv));
    const OCar* ego = &w->cars[base + obsIdx];
    const int flip = !ego->in.hasFlipped && !ego->in.hasDoubleJumped && ego->in.airTimeSinceJump < K_DOUBLEJUMP_MAX_DELAY;
    o[k++] = (float)flip;
    o[k++] = flip ? o_max(0.f, K_DOUBLEJUMP_MAX_DELAY - ego->in.airTimeSinceJump) : 0.f;
    o[k++] = (float)ego->in.hasJumped;
    o[k++] = (float)ego->in.isJumping;
    o[k++] = (float)ego->in.isFlipping;
    o[k++] = ego->in.flipTime;
    o[k++] = ego->demoTimer;
    if (e->prevControls) {
        o[k++] = ego->ctrl.throttle; o[k++] = ego->ctrl.steer; o[k++] = ego->ctrl.yaw;
        o[k++] = ego->ctrl.pitch; o[k++] = ego->ctrl.roll;
        o[k++] = (float)ego->ctrl.jump; o[k++] = (float)ego->ctrl.boost; o[k++] = (float)ego->ctrl.slide;
    }
    if (!e->normalize) return;
    /* normalizeObservations (Observations.cuh:240-317) */
    const float scale[3] = { 4108.f, 6000.f, 2076.f };
    for (int a = 0; a < 3; a++) o[a] /= scale[a];
    for (int a = 3; a < 6; a++) o[a] /= K_BALL_MAX_SPEED;
    for (int a = 6; a < 9; a++) o[a] /= K_BALL_MAX_ANG;
    for (int c = 0; c < nC; c++) {
        const int off = 9 + c * OBS_PER_CAR;
        for (int a = 0; a < 3; a++) o[off + a] /= scale[a];
        for (int a = 3; a < 6; a++) o[off + a] /= K_CAR_MAX_SPEED;
        for (int a = 6; a < 9; a++) o[off + a] /= K_CAR_MAX_ANG;
        o[off + 15] /= K_BOOST_MAX;
    }
    const int dOff = 9 + nC * OBS_PER_CAR + N_PADS;
    for (int p = 0; p < N_PADS; p++) o[dOff + p] /= 14692.54f;
    int r = dOff + N_PADS;
    for (int a = 0; a < 3; a++) {
        o[r + a] /= 2.f * scale[a];
        o[r + 3 + a] /= K_BALL_MAX_SPEED + K_CAR_MAX_SPEED;
    }
    r += 6;
    for (int c = 1; c < nC; c++) {
        for (int a = 0; a < 3; a++) {
            o[r + a] /= 2.f * scale[a];
            o[r + 3 + a] /= 2.f * K_CAR_MAX_SPEED;
        }
        r += 6;
    }
    for (int g = 0; g < 2; g++)
        for (int a = 0; a < 3; a++) o[r + g * 3 + a] /= 2.f * scale[a];
}

static void pack_obs(OEnv* e, float* out, const uint8_t* mask)
{
    const int nC = e->w.nCars;
    for (int s = 0; s < e->w.nSim; s++) {
        if (mask && !mask[s]) continue;
        for (int c = 0; c < nC; c++) pack_observation(e, s, c, out + ((size_t)s * nC + c) * e->obsDim);
    }
}

/* include/Physics/Observations.cuh:320-356 */
static void pack_state(OEnv* e, float* out, int touchWindow, const uint8_t* mask)
{
    const OWorld* w = &e->w;
    for (int s = 0; s < w->nSim; s++) {
        if (mask && !mask[s]) continue;
        float* o = out + (size_t)s * e->stateDim;
        int k = 0;
        put3(o, &k, w->sims[s].pos);
        put3(o, &k, w->sims[s].vel);
        put3(o, &k, w->sims[s].ang);
        for (int c = 0; c < w->nCars; c++) {
            const int ci = s * w->nCars + c;
            pack_car(w, ci, 0, o, &k);
            o[k++] = w->cars[ci].ballContactTick > w->tickCount - touchWindow;
        }
        for (int p = 0; p < N_PADS; p++) o[k++] = w->sims[s].pads[p] <= 0.f;
    }
}

/* include/Physics/Observations.cuh:360-397 and src/EnvIO.cu:466-484 */
static void pack_rewards_dones(OEnv* e)
{
    const OWorld* w = &e->w;
    for (int s = 0; s < w->nSim; s++) {
        const OSim* g = &w->sims[s];
        e->rewards[s] = (float)g->lastScorer;
        const int regExpired = g->episodeTicks >= e->maxTicks && g->blue != g->orange;
        const int otExpired = g->overtime && g->episodeTicks >= e->maxTicks + e->overtimeTicks;
        const int scored = g->lastScorer != 0;
        const int gameOver = !g->overtime && regExpired;
        const int timeout = e->noTouchTicks > 0 && w->tickCount - g->lastTouch >= e->noTouchTicks;
        e->dones[s] = gameOver || otExpired || timeout || scored;
        e->tscore[s] = g->blue - g->orange;
        e->tticks[s] = g->episodeTicks;
        e->tovertime[s] = (uint8_t)(g->overtime != 0);
    }
}

static void pack_raw_match(OEnv* e, const uint8_t* mask)
{
    for (int s = 0; s < e->w.nSim; s++) {
        if (mask && !mask[s]) continue;
        const OSim* g = &e->w.sims[s];
        e->score[s] = g->blue - g->orange;
        e->ticks[s] = g->episodeTicks;
        e->overtime[s] = (uint8_t)(g->overtime != 0);
    }
}

static void initial_packs(OEnv* e)
{
    pack_obs(e, e->obs, NULL);
    pack_state(e, e->state, 1, NULL);
    pack_state(e, e->tstate, 1, NULL);
    pack_rewards_dones(e);
    pack_raw_match(e, NULL);
}

/* ---------------------------------------------------------------- lifecycle */

OEnv* oracle_create(int nSim, int nBlue, int nOrange, int seed, int frameskip, int flags,
                    const char* objPath, char* err, int errLen)
{
    OArena* a = oarena_load(objPath, err, errLen);
    if (!a) return NULL;
    /* native mesh metadata, when named (src/ArenaMesh.cu:69-99) */
    const char* meta = getenv("CARL_ARENA_METADATA");
    if (meta && !oarena_load_metadata(a, meta, err, errLen)) {
        oarena_free(a);
        return NULL;
    }
    OEnv* e = (OEnv*)calloc(1, sizeof(OEnv));
    OWorld* w = &e->w;
    w->nSim = nSim; w->nBlue = nBlue; w->nOrange = nOrange; w->nCars = nBlue + nOrange;
    w->nTotal = nSim * w->nCars; w->seed = seed; w->arena = a;
    w->cars = (OCar*)calloc((size_t)w->nTotal, sizeof(OCar));
    w->sims = (OSim*)calloc((size_t)nSim, sizeof(OSim));
    e->frameskip = frameskip;
    e->invert = (flags & CARL_FLAG_INVERT_ORANGE) != 0;
    e->normalize = (flags & CARL_FLAG_NORMALIZE) != 0;
    e->prevControls = (flags & CARL_FLAG_PREVIOUS_CONTROLS) != 0;
    e->maxTicks = K_REGULATION_TICKS;
    e->overtimeTicks = K_REGULATION_TICKS;
    e->noTouchTicks = 0;
    e->obsDim = obs_dim(w->nCars, e->prevControls);
    e->stateDim = 9 + w->nCars * STATE_PER_CAR + N_PADS;
    const size_t nObs = (size_t)w->nTotal * e->obsDim;
    e->obs = (float*)calloc(nObs, 4);
    e->tobs = (float*)calloc(nObs, 4);
    e->state = (float*)calloc((size_t)nSim * e->stateDim, 4);
    e->tstate = (float*)calloc((size_t)nSim * e->stateDim, 4);
    e->rewards = (float*)calloc((size_t)nSim, 4);
    e->dones = (uint8_t*)calloc((size_t)nSim, 1);
    e->overtime = (uint8_t*)calloc((size_t)nSim, 1);
    e->tovertime = (uint8_t*)calloc((size_t)nSim, 1);
    e->score = (int32_t*)calloc((size_t)nSim, 4);
    e->ticks = (int32_t*)calloc((size_t)nSim, 4);
    e->tscore = (int32_t*)calloc((size_t)nSim, 4);
    e->tticks = (int32_t*)calloc((size_t)nSim, 4);
    e->actions = (int32_t*)calloc((size_t)w->nTotal * 7, 4);
    e->cactions = (float*)calloc((size_t)w->nTotal * 7, 4);
    ophys_reset_all(w);
    initial_packs(e);
    return e;
}

void oracle_destroy(OEnv* e)
{
    if (!e) return;
    oarena_free(e->w.arena);
    free(e->w.cars); free(e->w.sims);
    free(e->obs); free(e->tobs); free(e->state); free(e->tstate); free(e->rewards);
    free(e->dones); free(e->overtime); free(e->tovertime);
    free(e->score); free(e->ticks); free(e->tscore); free(e->tticks);
    free(e->actions); free(e->cactions);
    free(e);
}

void oracle_tick(OEnv* e, int kind, const void* actions, int n)
{
    for (int t = 0; t < n; t++) ophys_tick(&e->w, kind, actions);
}

void oracle_reset_dones(OEnv* e)
{
    for (int s = 0; s < e->w.nSim; s++)
        ophys_reset_after_done(&e->w, s, e->maxTicks, e->overtimeTicks, e->noTouchTicks);
}

/* python/carl.cu:320-370 */
void oracle_step(OEnv* e, int kind, const void* actions)
{
    const size_t n = (size_t)e->w.nTotal * 7 * 4;
    const void* src = actions;
    if (kind == 0) { memcpy(e->actions, actions, n); src = e->actions; }
    else if (kind == 1) { memcpy(e->cactions, actions, n); src = e->cactions; }
    oracle_tick(e, kind, src, e->frameskip);
    pack_rewards_dones(e);
    pack_state(e, e->tstate, e->frameskip, NULL);
    pack_obs(e, e->tobs, e->dones);
    oracle_reset_dones(e);
    pack_raw_match(e, NULL);
    pack_obs(e, e->obs, NULL);
    pack_state(e, e->state, 1, NULL);
}

void oracle_reset(OEnv* e)
{
    ophys_reset_all(&e->w);
    initial_packs(e);
}

/* ------------------------------------------------------------------ setters */

static int target_of(const OEnv* e, const int64_t* idx, int r)
{
    const int64_t t = idx ? idx[r] : r;
    if (t < 0 || t >= e->w.nSim) return -1;
    return (int)t;
}

/* src/EnvIO.cu:137-161 */
static void set_ball_rows(OEnv* e, const float* pos, const float* vel, const float* ang,
                          const int64_t* idx, int n, const uint8_t* mask)
{
    for (int r = 0; r < n; r++) {
        if (mask && !mask[r]) continue;
        const int t = target_of(e, idx, r);
        if (t < 0) continue;
        OSim* s = &e->w.sims[t];
        s->pos = v3(pos[3 * r], pos[3 * r + 1], pos[3 * r + 2]);
        s->vel = v3(vel[3 * r], vel[3 * r + 1], vel[3 * r + 2]);
        s->ang = v3(ang[3 * r], ang[3 * r + 1], ang[3 * r + 2]);
        s->imp = V_ZERO;
    }
}

/* src/EnvIO.cu:163-318 and 603-643 */
static void set_car_rows(OEnv* e, const float* pos, const float* rot, const float* vel,
                         const float* ang, const void* demoed, int byteDemoed,
                         const float* boost, const float* internal, const int64_t* idx,
                         int n, const uint8_t* mask)
{
    OWorld* w = &e->w;
    const int nC = w->nCars;
    for (int src = 0; src < n * nC; src++) {
        const int r = src / nC;
        if (mask && !mask[r]) continue;
        const int t = target_of(e, idx, r);
        if (t < 0) continue;
        const int local = src % nC;
        OCar* c = &w->cars[t * nC + local];
        const float prevBoost = c->in.boost;
        const int dm = byteDemoed ? ((const uint8_t*)demoed)[src] : ((const int32_t*)demoed)[src];
        c->pos = v3(pos[3 * src], pos[3 * src + 1], pos[3 * src + 2]);
        c->rot = q4(rot[4 * src], rot[4 * src + 1], rot[4 * src + 2], rot[4 * src + 3]);
        c->vel = v3(vel[3 * src], vel[3 * src + 1], vel[3 * src + 2]);
        c->ang = v3(ang[3 * src], ang[3 * src + 1], ang[3 * src + 2]);
        c->cen = vadd(c->pos, qworld(c->rot, K_CAR_OFFSETS));
        c->imp = V_ZERO;
        c->demoed = dm != 0;
        c->demoTimer = dm ? K_DEMO_RESPAWN_TIME + K_DT : 0.f;
        c->contactIdx = -1; c->contactCooldown = 0.f;
        c->ballHitTick = -1; c->ballContactTick = -1;
        memset(&c->ctrl, 0, sizeof c->ctrl);
        if (internal) {
            const float* v = internal + (size_t)src * 19;
            OInternal in;
            memset(&in, 0, sizeof in);
            in.onGround = v[0] != 0.f;
            in.airTimeSinceJump = v[1];
            in.handbrake = v[2];
            in.hasJumped = v[3] != 0.f;
            in.isJumping = v[4] != 0.f;
            in.lastJump = v[5] != 0.f;
            in.jumpTime = v[6];
            in.hasDoubleJumped = v[7] != 0.f;
            in.hasFlipped = v[8] != 0.f;
            in.isFlipping = v[9] != 0.f;
            in.flipTime = v[10];
            in.isAutoFlipping = v[11] != 0.f;
            in.autoFlipTimer = v[12];
            in.autoFlipScale = v[13];
            in.flipTorque = v3(v[14], v[15], v[16]);
            in.isBoosting = v[17] != 0.f;
            in.boostingTime = v[18];
            in.boost = boost ? o_min(K_BOOST_MAX, o_max(0.f, boost[src])) : prevBoost;
            c->in = in;
        } else if (boost) {
            c->in.boost = o_min(K_BOOST_MAX, o_max(0.f, boost[src]));
        }
        c->ctrl.jump = c->in.lastJump;
        c->brake = c->brakePrev = c->throttleVal = c->rawThrottle = 0.f;
        c->handbrakeVal = internal ? internal[(size_t)src * 19 + 2] : 0.f;
        c->steer = 0.f;
        c->jumpImp = V_ZERO;
        c->drive = c->drivePrev = 0.f;
        c->numTris = 0; c->hitCount = 0; c->manCount = 0;
        for (int k = 0; k < N_WHEELS; k++) { c->wheelContact[k] = 0; c->latF[k] = 0.f; c->lonF[k] = 0.f; }
    }
    /* refresh restored contacts once every pose is installed */
    for (int src = 0; src < n * nC; src++) {
        const int r = src / nC;
        if (mask && !mask[r]) continue;
        const int t = target_of(e, idx, r);
        if (t < 0) continue;
        const int ci = t * nC + src % nC;
        OCar* c = &w->cars[ci];
        if (c->demoed) {
            ophys_init_empty_wheels(c, V_Z);
            c->in.onGround = 0;
            continue;
        }
        ophys_broadphase(w, ci);
        ophys_raycast(w, ci);
        int cnt = 0;
        for (int k = 0; k < N_WHEELS; k++) cnt += c->wheelContact[k] != 0;
        c->in.onGround = cnt >= 3;
    }
}

static void set_match_rows(OEnv* e, const int32_t* blue, const int32_t* orange, const int32_t* ticks,
                           const int64_t* idx, int n, const uint8_t* mask)
{
    for (int r = 0; r < n; r++) {
        if (mask && !mask[r]) continue;
        const int t = target_of(e, idx, r);
        if (t < 0) continue;
        OSim* s = &e->w.sims[t];
        s->blue = blue[r]; s->orange = orange[r]; s->lastScorer = 0; s->overtime = 0;
        s->episodeTicks = ticks[r];
    }
}

static void reset_pad_rows(OEnv* e, const int64_t* idx, int n, const uint8_t* mask)
{
    for (int r = 0; r < n; r++) {
        if (mask && !mask[r]) continue;
        const int t = target_of(e, idx, r);
        if (t < 0) continue;
        for (int p = 0; p < N_PADS; p++) e->w.sims[t].pads[p] = 0.f;
    }
}

void oracle_set_ball(OEnv* e, const float* pos, const float* vel, const float* ang, const int64_t* idx, int n)
{
    if (n < 0) n = e->w.nSim;
    if (n > 0) set_ball_rows(e, pos, vel, ang, idx, n, NULL);
    pack_obs(e, e->obs, NULL);
    pack_state(e, e->state, 1, NULL);
    pack_state(e, e->tstate, 1, NULL);
}

void oracle_set_car(OEnv* e, const float* pos, const float* rot, const float* vel, const float* ang,
                    const void* demoed, int byteDemoed, const float* boost, const float* internal,
                    const int64_t* idx, int n)
{
    if (n < 0) n = e->w.nSim;
    if (n > 0) set_car_rows(e, pos, rot, vel, ang, demoed, byteDemoed, boost, internal, idx, n, NULL);
    pack_obs(e, e->obs, NULL);
    pack_state(e, e->state, 1, NULL);
    pack_state(e, e->tstate, 1, NULL);
}

void oracle_apply_reset(OEnv* e, const float* bpos, const float* bvel, const float* bang,
                        const float* cpos, const float* crot, const float* cvel, const float* cang,
                        const void* demoed, int byteDemoed, const float* boost, const float* internal,
                        const int32_t* blue, const int32_t* orange, const int32_t* ticks,
                        const int64_t* idx, int n, const uint8_t* mask)
{
    if (n == 0) return;
    reset_pad_rows(e, idx, n, mask);
    set_ball_rows(e, bpos, bvel, bang, idx, n, mask);
    set_car_rows(e, cpos, crot, cvel, cang, demoed, byteDemoed, boost, internal, idx, n, mask);
    if (blue) set_match_rows(e, blue, orange, ticks, idx, n, mask);
    pack_obs(e, e->obs, mask);
    pack_state(e, e->state, 1, mask);
    pack_raw_match(e, mask);
}

void oracle_set_match(OEnv* e, const int32_t* blue, const int32_t* orange, const int32_t* ticks,
                      const int64_t* idx, int n)
{
    if (n < 0) n = e->w.nSim;
    if (n > 0) set_match_rows(e, blue, orange, ticks, idx, n, NULL);
}

void oracle_reset_pads(OEnv* e, const int64_t* idx, int n)
{
    if (n < 0) n = e->w.nSim;
    if (n > 0) reset_pad_rows(e, idx, n, NULL);
}

int oracle_set_param(OEnv* e, int p, int v)
{
    switch (p) {
    case CARL_PARAM_MAX_TICKS: if (v < 1) return -1; e->maxTicks = v; return 0;
    case CARL_PARAM_OVERTIME_TIMEOUT_TICKS: if (v < 1) return -1; e->overtimeTicks = v; return 0;
    case CARL_PARAM_NO_TOUCH_TIMEOUT_TICKS: if (v < 0) return -1; e->noTouchTicks = v; return 0;
    case CARL_PARAM_FRAMESKIP: if (v < 1) return -1; e->frameskip = v; return 0;
    default: return -1;
    }
}

int oracle_get_param(OEnv* e, int p)
{
    switch (p) {
    case CARL_PARAM_MAX_TICKS: return e->maxTicks;
    case CARL_PARAM_OVERTIME_TIMEOUT_TICKS: return e->overtimeTicks;
    case CARL_PARAM_NO_TOUCH_TIMEOUT_TICKS: return e->noTouchTicks;
    case CARL_PARAM_FRAMESKIP: return e->frameskip;
    case CARL_PARAM_N_SIM: return e->w.nSim;
    case CARL_PARAM_N_CARS: return e->w.nCars;
    case CARL_PARAM_OBS_DIM: return e->obsDim;
    case CARL_PARAM_ACT_DIM: return e->w.nCars * 7;
    case CARL_PARAM_STATE_DIM: return e->stateDim;
    case CARL_PARAM_TICK_COUNT: return e->w.tickCount;
    case CARL_PARAM_N_BLUE: return e->w.nBlue;
    default: return -1;
    }
}

long oracle_buffer(OEnv* e, int id, void** data)
{
    const long nS = e->w.nSim, nA = (long)e->w.nTotal;
    switch (id) {
    case CARL_BUF_OBS: *data = e->obs; return nA * e->obsDim;
    case CARL_BUF_TRANSITION_OBS: *data = e->tobs; return nA * e->obsDim;
    case CARL_BUF_STATE: *data = e->state; return nS * e->stateDim;
    case CARL_BUF_TRANSITION_STATE: *data = e->tstate; return nS * e->stateDim;
    case CARL_BUF_ACTIONS: *data = e->actions; return nA * 7;
    case CARL_BUF_CONTINUOUS_ACTIONS: *data = e->cactions; return nA * 7;
    case CARL_BUF_REWARDS: *data = e->rewards; return nS;
    case CARL_BUF_DONES: *data = e->dones; return nS;
    case CARL_BUF_SCORE_DIFFERENCE: *data = e->score; return nS;
    case CARL_BUF_EPISODE_TICKS: *data = e->ticks; return nS;
    case CARL_BUF_TRANSITION_SCORE_DIFFERENCE: *data = e->tscore; return nS;
    case CARL_BUF_TRANSITION_EPISODE_TICKS: *data = e->tticks; return nS;
    case CARL_BUF_OVERTIME: *data = e->overtime; return nS;
    case CARL_BUF_TRANSITION_OVERTIME: *data = e->tovertime; return nS;
    default: *data = NULL; return -1;
    }
}

/* -------------------------------------------------------- export / import */

static uint32_t fb(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }
static float bf(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }
static uint32_t ib(int i) { return (uint32_t)i; }

#define CF(field, car) car_state[(size_t)(field) * nT + (car)]
#define SF(field, sim) sim_state[(size_t)(field) * nS + (sim)]

void oracle_export(OEnv* e, uint32_t* car_state, uint32_t* sim_state, int* tick)
{
    const OWorld* w = &e->w;
    const size_t nT = (size_t)w->nTotal, nS = (size_t)w->nSim;
    for (size_t i = 0; i < nT; i++) {
        const OCar* c = &w->cars[i];
        const float v[] = { c->pos.x, c->pos.y, c->pos.z, c->vel.x, c->vel.y, c->vel.z,
                            c->ang.x, c->ang.y, c->ang.z, c->rot.x, c->rot.y, c->rot.z, c->rot.w,
                            c->cen.x, c->cen.y, c->cen.z, c->imp.x, c->imp.y, c->imp.z };
        for (int f = 0; f < 19; f++) CF(f, i) = fb(v[f]);
        CF(CARL_CAR_DEMOED, i) = ib(c->demoed);
        CF(CARL_CAR_DEMO_TIMER, i) = fb(c->demoTimer);
        CF(CARL_CAR_CONTACT_IDX, i) = ib(c->contactIdx);
        CF(CARL_CAR_CONTACT_COOLDOWN, i) = fb(c->contactCooldown);
        CF(CARL_CAR_BALL_HIT_TICK, i) = ib(c->ballHitTick);
        CF(CARL_CAR_BALL_CONTACT_TICK, i) = ib(c->ballContactTick);
        CF(CARL_CAR_ARENA_CONTACT_TICK, i) = ib(c->arenaContactTick);
        for (int k = 0; k < 4; k++) {
            CF(CARL_CAR_WHEEL_SOURCE + k, i) = ib(c->wheelSource[k]);
            CF(CARL_CAR_WHEEL_CONTACT + k, i) = ib(c->wheelContact[k]);
            CF(CARL_CAR_LAT_FRICTION + k, i) = fb(c->latF[k]);
            CF(CARL_CAR_LON_FRICTION + k, i) = fb(c->lonF[k]);
        }
        CF(CARL_CAR_CTRL_THROTTLE, i) = fb(c->ctrl.throttle);
        CF(CARL_CAR_CTRL_STEER, i) = fb(c->ctrl.steer);
        CF(CARL_CAR_CTRL_YAW, i) = fb(c->ctrl.yaw);
        CF(CARL_CAR_CTRL_PITCH, i) = fb(c->ctrl.pitch);
        CF(CARL_CAR_CTRL_ROLL, i) = fb(c->ctrl.roll);
        CF(CARL_CAR_CTRL_JUMP, i) = ib(c->ctrl.jump);
        CF(CARL_CAR_CTRL_BOOST, i) = ib(c->ctrl.boost);
        CF(CARL_CAR_CTRL_SLIDE, i) = ib(c->ctrl.slide);
        const OInternal* n = &c->in;
        CF(CARL_CAR_ON_GROUND, i) = ib(n->onGround);
        CF(CARL_CAR_AIR_TIME, i) = fb(n->airTime);
        CF(CARL_CAR_AIR_TIME_SINCE_JUMP, i) = fb(n->airTimeSinceJump);
        CF(CARL_CAR_HANDBRAKE, i) = fb(n->handbrake);
        CF(CARL_CAR_HAS_JUMPED, i) = ib(n->hasJumped);
        CF(CARL_CAR_IS_JUMPING, i) = ib(n->isJumping);
        CF(CARL_CAR_JUMP_TIME, i) = fb(n->jumpTime);
        CF(CARL_CAR_LAST_JUMP, i) = ib(n->lastJump);
        CF(CARL_CAR_HAS_DOUBLE_JUMPED, i) = ib(n->hasDoubleJumped);
        CF(CARL_CAR_HAS_FLIPPED, i) = ib(n->hasFlipped);
        CF(CARL_CAR_IS_FLIPPING, i) = ib(n->isFlipping);
        CF(CARL_CAR_FLIP_TIME, i) = fb(n->flipTime);
        CF(CARL_CAR_IS_AUTO_FLIPPING, i) = ib(n->isAutoFlipping);
        CF(CARL_CAR_AUTO_FLIP_TIMER, i) = fb(n->autoFlipTimer);
        CF(CARL_CAR_AUTO_FLIP_SCALE, i) = fb(n->autoFlipScale);
        CF(CARL_CAR_FLIP_TORQUE, i) = fb(n->flipTorque.x);
        CF(CARL_CAR_FLIP_TORQUE + 1, i) = fb(n->flipTorque.y);
        CF(CARL_CAR_FLIP_TORQUE + 2, i) = fb(n->flipTorque.z);
        CF(CARL_CAR_RESPAWN_IDX, i) = ib(n->respawnIdx);
        CF(CARL_CAR_LAST_RESPAWN_DIR, i) = ib(n->lastRespawnDir);
        CF(CARL_CAR_IS_BOOSTING, i) = ib(n->isBoosting);
        CF(CARL_CAR_BOOST, i) = fb(n->boost);
        CF(CARL_CAR_BOOSTING_TIME, i) = fb(n->boostingTime);
        CF(CARL_CAR_TIME_SINCE_BOOSTED, i) = fb(n->timeSinceBoosted);
        CF(CARL_CAR_BRAKE_STAGE, i) = fb(c->brake);
        CF(CARL_CAR_STEER_STAGE, i) = fb(c->steer);
        CF(CARL_CAR_DRIVE_STAGE, i) = fb(c->drive);
        CF(CARL_CAR_MANIFOLD_COUNT, i) = ib(c->manCount);
        CF(CARL_CAR_MANIFOLD_NORMAL, i) = fb(c->manNormal.x);
        CF(CARL_CAR_MANIFOLD_NORMAL + 1, i) = fb(c->manNormal.y);
        CF(CARL_CAR_MANIFOLD_NORMAL + 2, i) = fb(c->manNormal.z);
    }
    for (size_t s = 0; s < nS; s++) {
        const OSim* g = &w->sims[s];
        const V3 vs[8] = { g->pos, g->vel, g->ang, g->imp, g->intPos, g->intVel, g->expPos, g->expVel };
        for (int q = 0; q < 8; q++) {
            SF(3 * q, s) = fb(vs[q].x); SF(3 * q + 1, s) = fb(vs[q].y); SF(3 * q + 2, s) = fb(vs[q].z);
        }
        SF(CARL_SIM_BALL_INT_VALID, s) = ib(g->intValid);
        SF(CARL_SIM_BLUE_SCORE, s) = ib(g->blue);
        SF(CARL_SIM_ORANGE_SCORE, s) = ib(g->orange);
        SF(CARL_SIM_LAST_SCORER, s) = ib(g->lastScorer);
        SF(CARL_SIM_GOAL_TICK, s) = ib(g->goalTick);
        SF(CARL_SIM_OVERTIME, s) = ib(g->overtime);
        SF(CARL_SIM_EPISODE_TICKS, s) = ib(g->episodeTicks);
        SF(CARL_SIM_LAST_TOUCH_TICK, s) = ib(g->lastTouch);
        SF(CARL_SIM_BALL_ARENA_CONTACT_TICK, s) = ib(g->ballArenaContactTick);
        for (int p = 0; p < N_PADS; p++) SF(CARL_SIM_PAD_COOLDOWN + p, s) = fb(g->pads[p]);
    }
    if (tick) *tick = w->tickCount;
}

void oracle_import(OEnv* e, const uint32_t* car_state, const uint32_t* sim_state, int tick)
{
    OWorld* w = &e->w;
    const size_t nT = (size_t)w->nTotal, nS = (size_t)w->nSim;
    for (size_t i = 0; i < nT; i++) {
        OCar* c = &w->cars[i];
        float v[19];
        for (int f = 0; f < 19; f++) v[f] = bf(CF(f, i));
        c->pos = v3(v[0], v[1], v[2]); c->vel = v3(v[3], v[4], v[5]); c->ang = v3(v[6], v[7], v[8]);
        c->rot = q4(v[9], v[10], v[11], v[12]); c->cen = v3(v[13], v[14], v[15]); c->imp = v3(v[16], v[17], v[18]);
        c->demoed = (int)CF(CARL_CAR_DEMOED, i);
        c->demoTimer = bf(CF(CARL_CAR_DEMO_TIMER, i));
        c->contactIdx = (int)CF(CARL_CAR_CONTACT_IDX, i);
        c->contactCooldown = bf(CF(CARL_CAR_CONTACT_COOLDOWN, i));
        c->ballHitTick = (int)CF(CARL_CAR_BALL_HIT_TICK, i);
        c->ballContactTick = (int)CF(CARL_CAR_BALL_CONTACT_TICK, i);
        c->arenaContactTick = (int)CF(CARL_CAR_ARENA_CONTACT_TICK, i);
        for (int k = 0; k < 4; k++) {
            c->wheelSource[k] = (int)CF(CARL_CAR_WHEEL_SOURCE + k, i);
            c->wheelContact[k] = (int)CF(CARL_CAR_WHEEL_CONTACT + k, i);
            c->latF[k] = bf(CF(CARL_CAR_LAT_FRICTION + k, i));
            c->lonF[k] = bf(CF(CARL_CAR_LON_FRICTION + k, i));
        }
        c->ctrl.throttle = bf(CF(CARL_CAR_CTRL_THROTTLE, i));
        c->ctrl.steer = bf(CF(CARL_CAR_CTRL_STEER, i));
        c->ctrl.yaw = bf(CF(CARL_CAR_CTRL_YAW, i));
        c->ctrl.pitch = bf(CF(CARL_CAR_CTRL_PITCH, i));
        c->ctrl.roll = bf(CF(CARL_CAR_CTRL_ROLL, i));
        c->ctrl.jump = (int)CF(CARL_CAR_CTRL_JUMP, i);
        c->ctrl.boost = (int)CF(CARL_CAR_CTRL_BOOST, i);
        c->ctrl.slide = (int)CF(CARL_CAR_CTRL_SLIDE, i);
        OInternal* n = &c->in;
        n->onGround = (int)CF(CARL_CAR_ON_GROUND, i);
        n->airTime = bf(CF(CARL_CAR_AIR_TIME, i));
        n->airTimeSinceJump = bf(CF(CARL_CAR_AIR_TIME_SINCE_JUMP, i));
        n->handbrake = bf(CF(CARL_CAR_HANDBRAKE, i));
        n->hasJumped = (int)CF(CARL_CAR_HAS_JUMPED, i);
        n->isJumping = (int)CF(CARL_CAR_IS_JUMPING, i);
        n->jumpTime = bf(CF(CARL_CAR_JUMP_TIME, i));
        n->lastJump = (int)CF(CARL_CAR_LAST_JUMP, i);
        n->hasDoubleJumped = (int)CF(CARL_CAR_HAS_DOUBLE_JUMPED, i);
        n->hasFlipped = (int)CF(CARL_CAR_HAS_FLIPPED, i);
        n->isFlipping = (int)CF(CARL_CAR_IS_FLIPPING, i);
        n->flipTime = bf(CF(CARL_CAR_FLIP_TIME, i));
        n->isAutoFlipping = (int)CF(CARL_CAR_IS_AUTO_FLIPPING, i);
        n->autoFlipTimer = bf(CF(CARL_CAR_AUTO_FLIP_TIMER, i));
        n->autoFlipScale = bf(CF(CARL_CAR_AUTO_FLIP_SCALE, i));
        n->flipTorque = v3(bf(CF(CARL_CAR_FLIP_TORQUE, i)), bf(CF(CARL_CAR_FLIP_TORQUE + 1, i)),
                           bf(CF(CARL_CAR_FLIP_TORQUE + 2, i)));
        n->respawnIdx = (int)CF(CARL_CAR_RESPAWN_IDX, i);
        n->lastRespawnDir = (int)CF(CARL_CAR_LAST_RESPAWN_DIR, i);
        n->isBoosting = (int)CF(CARL_CAR_IS_BOOSTING, i);
        n->boost = bf(CF(CARL_CAR_BOOST, i));
        n->boostingTime = bf(CF(CARL_CAR_BOOSTING_TIME, i));
        n->timeSinceBoosted = bf(CF(CARL_CAR_TIME_SINCE_BOOSTED, i));
        c->brake = bf(CF(CARL_CAR_BRAKE_STAGE, i));
        c->steer = bf(CF(CARL_CAR_STEER_STAGE, i));
        c->drive = bf(CF(CARL_CAR_DRIVE_STAGE, i));
        c->manCount = (int)CF(CARL_CAR_MANIFOLD_COUNT, i);
        c->manNormal = v3(bf(CF(CARL_CAR_MANIFOLD_NORMAL, i)), bf(CF(CARL_CAR_MANIFOLD_NORMAL + 1, i)),
                          bf(CF(CARL_CAR_MANIFOLD_NORMAL + 2, i)));
        c->jumpImp = V_ZERO; c->angImp = V_ZERO;
    }
    for (size_t s = 0; s < nS; s++) {
        OSim* g = &w->sims[s];
        V3* vs[8] = { &g->pos, &g->vel, &g->ang, &g->imp, &g->intPos, &g->intVel, &g->expPos, &g->expVel };
        for (int q = 0; q < 8; q++) *vs[q] = v3(bf(SF(3 * q, s)), bf(SF(3 * q + 1, s)), bf(SF(3 * q + 2, s)));
        g->intValid = (int)SF(CARL_SIM_BALL_INT_VALID, s);
        g->blue = (int)SF(CARL_SIM_BLUE_SCORE, s);
        g->orange = (int)SF(CARL_SIM_ORANGE_SCORE, s);
        g->lastScorer = (int)SF(CARL_SIM_LAST_SCORER, s);
        g->goalTick = (int)SF(CARL_SIM_GOAL_TICK, s);
        g->overtime = (int)SF(CARL_SIM_OVERTIME, s);
        g->episodeTicks = (int)SF(CARL_SIM_EPISODE_TICKS, s);
        g->lastTouch = (int)SF(CARL_SIM_LAST_TOUCH_TICK, s);
        g->ballArenaContactTick = (int)SF(CARL_SIM_BALL_ARENA_CONTACT_TICK, s);
        for (int p = 0; p < N_PADS; p++) g->pads[p] = bf(SF(CARL_SIM_PAD_COOLDOWN + p, s));
    }
    w->tickCount = tick;
}

/* ------------------------------------------------------------ inspection */

int oracle_arena_counts(OEnv* e, int* nv, int* nt, int* nr)
{
    *nv = e->w.arena->nVerts; *nt = e->w.arena->nTris; *nr = e->w.arena->cellPrefix[N_CELLS];
    return N_CELLS;
}

void oracle_arena_copy(OEnv* e, float* verts, int32_t* tris, float* angles, int32_t* prefix, int32_t* cellTris)
{
    const OArena* a = e->w.arena;
    for (int i = 0; i < a->nVerts; i++) { verts[3 * i] = a->verts[i].x; verts[3 * i + 1] = a->verts[i].y; verts[3 * i + 2] = a->verts[i].z; }
    for (int i = 0; i < 3 * a->nTris; i++) tris[i] = a->tris[i];
    for (int i = 0; i < a->nTris; i++) { angles[3 * i] = a->angs[i].x; angles[3 * i + 1] = a->angs[i].y; angles[3 * i + 2] = a->angs[i].z; }
    for (int i = 0; i <= N_CELLS; i++) prefix[i] = a->cellPrefix[i];
    for (int i = 0; i < a->cellPrefix[N_CELLS]; i++) cellTris[i] = a->cellTris[i];
}

void oracle_cell_of(float x, float y, float z, int* c3) { oarena_cell3(v3(x, y, z), &c3[0], &c3[1], &c3[2]); }

void oracle_broadphase(OEnv* e, int32_t* cell, int32_t* count)
{
    for (int c = 0; c < e->w.nTotal; c++) {
        ophys_broadphase(&e->w, c);
        cell[c] = e->w.cars[c].cellIdx;
        count[c] = e->w.cars[c].numTris;
    }
}

void oracle_raycast(OEnv* e, float* dist, float* normal, int32_t* source)
{
    for (int c = 0; c < e->w.nTotal; c++) ophys_broadphase(&e->w, c);
    for (int c = 0; c < e->w.nTotal; c++) {
        OCar* car = &e->w.cars[c];
        /* the raycast writes wheel contact outputs; keep the persistent copy */
        int src[4], con[4];
        memcpy(src, car->wheelSource, sizeof src);
        memcpy(con, car->wheelContact, sizeof con);
        ophys_raycast(&e->w, c);
        for (int k = 0; k < 4; k++) {
            dist[4 * c + k] = car->rayDist[k];
            normal[12 * c + 3 * k] = car->rayNormal[k].x;
            normal[12 * c + 3 * k + 1] = car->rayNormal[k].y;
            normal[12 * c + 3 * k + 2] = car->rayNormal[k].z;
            source[4 * c + k] = car->wheelSource[k];
        }
        memcpy(car->wheelSource, src, sizeof src);
        memcpy(car->wheelContact, con, sizeof con);
    }
}

int oracle_ball_contacts(OEnv* e, const float* center, int32_t* tri, float* point, float* normal, float* depth,
                         float* reduction)
{
    return ophys_probe_ball_contacts(&e->w, center, tri, point, normal, depth, reduction);
}

/* ------------------------------------------------------------------ probes */

int oracle_ball_hit_prev_tick(int h, int t) { return ophys_ball_hit_prev_tick(h, t); }
float oracle_probe_ball_floor_split(float d, float v, int hit) { return ophys_probe_ball_floor_split(d, v, hit); }
void oracle_probe_dodge(float p, float y, float r, int* hf, int* hd, float* vel) { ophys_probe_dodge(p, y, r, hf, hd, vel); }
void oracle_probe_autoflip(const float* q, int j, int n, const float* nrm, int* af, float* t, float* a)
{
    ophys_probe_autoflip(q, j, n, nrm, af, t, a);
}
void oracle_probe_steer_stage(float s, float* p, float* c) { ophys_probe_steer_stage(s, p, c); }
int oracle_kickoff_perm(int i, int s) { return ophys_kickoff_perm(i, s); }
void oracle_probe_box_tri_sat(const float* t, int* o, int* a, float* d, float* ax) { ophys_probe_box_tri_sat(t, o, a, d, ax); }
int oracle_probe_box_tri_contacts(const float* t, int* a, float* cp, float* ap, float* n, float* d)
{
    return ophys_probe_box_tri_contacts(t, a, cp, ap, n, d);
}
int oracle_probe_manifold(OEnv* e, int car, float* cp, float* wp, float* n, float* d)
{
    if (car < 0 || car >= e->w.nTotal) return -1;
    return ophys_probe_manifold(&e->w, car, cp, wp, n, d);
}
int oracle_probe_box_box_contacts(const float* ca, const float* ra, const float* cb, const float* rb, int* a,
                                  float* pa, float* pb, float* n, float* d)
{
    return ophys_probe_box_box_contacts(ca, ra, cb, rb, a, pa, pb, n, d);
}
void oracle_probe_box_box_sat(const float* ca, const float* ra, const float* cb, const float* rb, int* o, int* a,
                              float* d)
{
    ophys_probe_box_box_sat(ca, ra, cb, rb, o, a, d);
}
uint32_t oracle_hash32(uint32_t v) { return o_hash32(v); }
void oracle_sincos(float x, float* s, float* c) { o_sincos(x, s, c); }
float oracle_atan2(float y, float x) { return o_atan2(y, x); }
void oracle_integrate_quat(const float* r, const float* a, float* out)
{
    const Q4 q = ophys_integrate_quat(q4(r[0], r[1], r[2], r[3]), v3(a[0], a[1], a[2]));
    out[0] = q.x; out[1] = q.y; out[2] = q.z; out[3] = q.w;
}

/* ------------------------------------------------------- CPU throughput run */

typedef struct {
    OEnv* env;
    int ticks, seed;
    long done;
    double seconds;
} CpuJob;

static uint64_t splitmix(uint64_t* s)
{
    uint64_t z = (*s += 0x9e3779b97f4a7c15ull);
    z = (z ^ (z >> 30)) * 0xbf58476d1ce4e5b9ull;
    z = (z ^ (z >> 27)) * 0x94d049bb133111ebull;
    return z ^ (z >> 31);
}

static float uni(uint64_t* s) { return (float)((splitmix(s) >> 40) * (1.0 / 16777216.0)); }

static double now_seconds(void)
{
    struct timespec t;
    clock_gettime(CLOCK_MONOTONIC, &t);
    return (double)t.tv_sec + 1e-9 * (double)t.tv_nsec;
}

/* one 1v1 arena: direct controls (throttle/steer/pitch/yaw/roll U[-1,1],
 * jump/boost/handbrake Bernoulli(0.5)) resampled every 8 ticks */
static void* cpu_worker(void* arg)
{
    CpuJob* j = (CpuJob*)arg;
    OEnv* e = j->env;
    uint64_t rng = (uint64_t)j->seed * 0x9e3779b97f4a7c15ull + 1;
    carl_controls ctl[2];
    const double t0 = now_seconds();
    for (int t = 0; t < j->ticks; t++) {
        if (t % 8 == 0) {
            for (int c = 0; c < 2; c++) {
                ctl[c].throttle = 2.f * uni(&rng) - 1.f;
                ctl[c].steer = 2.f * uni(&rng) - 1.f;
                ctl[c].pitch = 2.f * uni(&rng) - 1.f;
                ctl[c].yaw = 2.f * uni(&rng) - 1.f;
                ctl[c].roll = 2.f * uni(&rng) - 1.f;
                ctl[c].jump = uni(&rng) < .5f;
                ctl[c].boost = uni(&rng) < .5f;
                ctl[c].slide = uni(&rng) < .5f;
            }
        }
        ophys_tick(&e->w, CARL_ACTIONS_DIRECT, ctl);
        oracle_reset_dones(e);
    }
    j->seconds = now_seconds() - t0;
    j->done = j->ticks;
    return NULL;
}

double oracle_cpu_throughput(const char* obj, int threads, int ticks, int seed)
{
    if (threads < 1) threads = 1;
    pthread_t* th = (pthread_t*)calloc((size_t)threads, sizeof(pthread_t));
    CpuJob* jobs = (CpuJob*)calloc((size_t)threads, sizeof(CpuJob));
    char err[128];
    for (int i = 0; i < threads; i++) {
        jobs[i].env = oracle_create(1, 1, 1, seed + i, 1, CARL_FLAG_INVERT_ORANGE, obj, err, sizeof err);
        if (!jobs[i].env) { threads = i; break; }
        jobs[i].ticks = ticks; jobs[i].seed = seed + i;
    }
    for (int i = 0; i < threads; i++) pthread_create(&th[i], NULL, cpu_worker, &jobs[i]);
    long total = 0;
    double slowest = 0.0;
    for (int i = 0; i < threads; i++) {
        pthread_join(th[i], NULL);
        total += jobs[i].done;
        if (jobs[i].seconds > slowest) slowest = jobs[i].seconds;
        oracle_destroy(jobs[i].env);
    }
    free(th); free(jobs);
    return slowest > 0 ? (double)total / slowest : 0.0;
}
