/*
 * ointernal.h - constants and data structures of the CPU oracle.
 *
 * TEST INFRASTRUCTURE (see omath.h).  Constants restate
 * include/RLConstants.cuh:1-278, include/Physics/BoostPads.cuh:14-56 and the
 * ball/contact constants of include/Physics/BallArena/Contact.cuh:28-37.
 * State structures follow include/State/GameState.cuh and
 * include/State/Workspace.cuh, laid out per car / per simulation (AoS), which
 * is the plain CPU form of the reference's structure-of-arrays.
 */
#ifndef CARL_ORACLE_INTERNAL_H
#define CARL_ORACLE_INTERNAL_H

#include "omath.h"

/* ---- math / arena ---- */
#define K_PI 3.14159265358979323846f
static const float K_PI_2 = K_PI / 2;
static const float K_PI_4 = K_PI / 4;
static const float K_SQRT_1_2 = 0.7071067811865475244f;
static const float K_FLT_EPS = 1.192092896e-07f;
#define K_FLT_MAX 3.402823466e+38f

static const V3 K_ARENA_MIN = { -4108.f, -6000.f, -14.f };
static const V3 K_ARENA_MAX = { 4108.f, 6000.f, 2076.f };
#define GRID_X 48
#define GRID_Y 48
#define GRID_Z 10
#define N_CELLS (GRID_X * GRID_Y * GRID_Z)
static const V3 K_GRID_DIMS = { 48.f, 48.f, 10.f };
/* CELL_SIZE = (ARENA_MAX - ARENA_MIN) / GRID_DIMS, evaluated in float */
#define K_CELL_X ((4108.f - -4108.f) / 48.f)
#define K_CELL_Y ((6000.f - -6000.f) / 48.f)
#define K_CELL_Z ((2076.f - -14.f) / 10.f)

#define K_BOUNDARY_EDGE_ANGLE (2.f * K_PI)

/* ---- car ---- */
static const V3 K_CAR_HALF = { 60.186455f, 43.282655f, 19.262505f };
#define K_CAR_SHAPE_MARGIN 1.932955f
static const V3 K_CAR_OFFSETS = { 13.87566f, 0.f, 20.755f };
#define K_CAR_REST_Z 17.f
#define K_CAR_RESPAWN_Z 36.f
#define K_BALL_REST_Z 93.15f
#define K_BALL_RADIUS 91.25f

#define N_PADS 34
#define K_BOOST_MAX 100.f
#define K_BOOST_SPAWN (K_BOOST_MAX / 3.f)

#define N_WHEELS 4
#define K_FRONT_WHEEL_RADIUS 12.5f
#define K_BACK_WHEEL_RADIUS 15.f
#define K_FRONT_SUSP_REST 26.755f
#define K_BACK_SUSP_REST 25.055f
#define K_MAX_SUSP_TRAVEL 12.f
#define K_SUSP_SUBTRACTION 2.5f
#define K_FRONT_SUSP_X 37.3743f
#define K_FRONT_SUSP_Y 25.9f
#define K_BACK_SUSP_X -47.6257f
#define K_BACK_SUSP_Y 29.5f
#define K_FRONT_RAY_LEN (K_FRONT_SUSP_REST + K_MAX_SUSP_TRAVEL + K_FRONT_WHEEL_RADIUS - K_SUSP_SUBTRACTION)
#define K_BACK_RAY_LEN (K_BACK_SUSP_REST + K_MAX_SUSP_TRAVEL + K_BACK_WHEEL_RADIUS - K_SUSP_SUBTRACTION)

enum { SRC_NONE = 0, SRC_ARENA = 1, SRC_CAR = 2, SRC_BALL = 3 };

#define MAX_TRI_PAIRS 32
#define MAX_PAIR_CONTACTS 8
#define MAX_MANIFOLD 4
#define K_ANG_MOTION_THRESH K_PI_4
#define K_WORLD_RESTITUTION 0.3f
#define K_WORLD_FRICTION 0.3f
#define K_CONTACT_BREAK 2.03122735f

#define K_TICKS_PER_SECOND 120
#define K_DT (1.f / K_TICKS_PER_SECOND)
#define K_REGULATION_TICKS (5 * 60 * K_TICKS_PER_SECOND)
#define K_CAR_MASS 180.f
#define K_CAR_INV_MASS (1.f / K_CAR_MASS)
#define K_CAR_MAX_SPEED 2300.f
#define K_CAR_MAX_ANG 5.5f
static const V3 K_CAR_INV_INERTIA = { 1.f / 134665.94f, 1.f / 239607.22f, 1.f / 329747.90f };
static const V3 K_GRAVITY = { 0.f, 0.f, -650.f };

#define K_SOLVER_ITERS 10
#define K_CONTACT_ERP 0.8f
#define K_WARMSTART 0.85f
#define K_LINEAR_SLOP 0.f
#define K_SPLIT_TURN_ERP 0.1f
#define K_SPLIT_PEN_THRESH 1.0e30f
#define K_RESTITUTION_VEL_THRESH 10.f

#define K_SUSP_STIFFNESS 500.f
#define K_SUSP_DAMP_COMP 25.f
#define K_SUSP_DAMP_RELAX 40.f
#define K_SUSP_SCALE_FRONT 35.75f
#define K_SUSP_SCALE_BACK 54.265f
#define K_SUSP_PUSHBACK_ERP 0.2f
#define K_SUSP_PUSHBACK_DT_FIRST (1.f / 60.f)
#define K_STOPPING_VEL 25.f
#define K_AUTOROLL_FORCE 100.f
#define K_AUTOROLL_TORQUE 80.f

#define K_JUMP_ACCEL (4375.f / 3.f)
#define K_JUMP_IMMEDIATE (875.f / 3.f)
#define K_JUMP_MIN_TIME 0.025f
#define K_JUMP_RESET_PAD (1.f / 40.f)
#define K_JUMP_MAX_TIME 0.2f
#define K_DOUBLEJUMP_MAX_DELAY 1.25f
#define K_FLIP_Z_DAMP_120 0.35f
#define K_FLIP_Z_DAMP_START 0.15f
#define K_FLIP_Z_DAMP_END 0.21f
#define K_FLIP_TORQUE_TIME 0.65f
#define K_FLIP_PITCHLOCK_EXTRA 0.3f
#define K_FLIP_INITIAL_VEL 500.f
#define K_FLIP_TORQUE_X 260.f
#define K_FLIP_TORQUE_Y 224.f
#define K_FLIP_FWD_SCALE 1.f
#define K_FLIP_SIDE_SCALE 1.9f
#define K_FLIP_BACK_SCALE 2.5f
#define K_FLIP_BACK_X (16.f / 15.f)
#define K_DODGE_DEADZONE 0.5f

#define K_THROTTLE_AIR_ACCEL (200.f / 3.f)
#define K_THROTTLE_GROUND_ACCEL 1600.f
#define K_THROTTLE_DEADZONE 0.001f
#define K_COASTING_BRAKE 0.15f
#define K_BOOST_PER_SECOND (K_BOOST_MAX / 3.f)
#define K_BOOST_MIN_TIME 0.1f
#define K_BOOST_ACCEL_GROUND (2975.f / 3.f)
#define K_BOOST_ACCEL_AIR (3175.f / 3.f)
#define K_POWERSLIDE_RISE 5.f
#define K_POWERSLIDE_FALL 2.f

#define K_TORQUE_SCALE (2.f * K_PI / 65536.f * 1000.f)
static const float K_AIR_TORQUE[3] = { 130.f, 95.f, 400.f };
static const float K_AIR_DAMPING[3] = { 30.f, 20.f, 50.f };
#define K_AUTOFLIP_IMPULSE 200.f
#define K_AUTOFLIP_TORQUE 50.f
#define K_AUTOFLIP_TIME 0.4f
#define K_AUTOFLIP_NORMZ 0.70710678f
#define K_AUTOFLIP_ROLL 2.8f

#define K_CARCAR_FRICTION 0.09f
#define K_CARCAR_RESTITUTION 0.1f
#define K_BUMP_COOLDOWN 0.25f
#define K_BUMP_MIN_FWD 64.5f
#define K_DEMO_RESPAWN_TIME 3.f
#define K_DEMO_INPUT_DEADZONE 0.5f
#define K_SUPERSONIC 2200.f

#define K_BALL_MASS (K_CAR_MASS / 6.f)
#define K_BALL_INV_MASS (1.f / K_BALL_MASS)
#define K_BALL_MAX_SPEED 6000.f
#define K_BALL_MAX_ANG 6.f
#define K_BALL_RESTITUTION 0.6f
#define K_BALL_FRICTION 0.35f
#define K_BALL_INERTIA (0.4f * K_BALL_MASS * K_BALL_RADIUS * K_BALL_RADIUS)
#define K_BALL_INV_INERTIA (1.f / K_BALL_INERTIA)
/* powf(1 - BALL_DRAG, PHYS_DT), correctly rounded (BALL_DRAG = 0.03) */
#define K_BALL_DRAG_FACTOR 0x1.ffdebcp-1f

#define K_CARBALL_RESTITUTION 0.f
#define K_CARBALL_FRICTION 2.f
#define K_CARBALL_BREAK 1.825f
#define K_CARBALL_MARGIN K_CAR_SHAPE_MARGIN
#define K_EXTRA_Z_SCALE 0.35f
#define K_EXTRA_FWD_SCALE 0.65f
#define K_EXTRA_MAXDV 4600.f

#define K_GOAL_CENTER_Y 5120.f
#define K_GOAL_CENTER_Z 321.3875f
#define K_GOAL_THRESHOLD_Y 5124.25f

#define K_BALL_ARENA_BREAK 1.905f
#define MAX_BALL_CONTACTS 68

/* boost pads */
#define K_SMALL_PAD_RADIUS 144.f
#define K_BIG_PAD_RADIUS 208.f
#define K_PAD_HEIGHT 95.f
#define K_SMALL_PAD_AMOUNT 12.f
#define K_BIG_PAD_AMOUNT 100.f
#define K_SMALL_PAD_COOLDOWN 4.f
#define K_BIG_PAD_COOLDOWN 10.f

/* ---- controls ---- */
typedef struct {
    float throttle, steer, yaw, pitch, roll;
    int jump, boost, slide;
} OControls;

typedef struct {
    int onGround;
    float airTime, airTimeSinceJump, handbrake;
    int hasJumped, isJumping;
    float jumpTime;
    int lastJump;
    int hasDoubleJumped, hasFlipped, isFlipping;
    float flipTime;
    int isAutoFlipping;
    float autoFlipTimer, autoFlipScale;
    V3 flipTorque;
    int respawnIdx, lastRespawnDir;
    int isBoosting;
    float boost, boostingTime, timeSinceBoosted;
} OInternal;

typedef struct {
    V3 v0, v1, v2;      /* car-local vertices */
    int tri;
    int axisIdx;
    V3 minAxis;
    float minPen;
} OHit;

typedef struct {
    V3 carPos, arenaPos, normal;
    float depth;
} OContact;

typedef struct {
    V3 carPos, worldPos, worldNormal;
    float dist, friction, restitution, impulse, impulseTan;
    int lifetime;
} OManPoint;

typedef struct {
    /* persistent */
    V3 pos, vel, ang, cen, imp;
    Q4 rot;
    int demoed;
    float demoTimer;
    int contactIdx;
    float contactCooldown;
    int ballHitTick, ballContactTick, arenaContactTick;
    int wheelSource[N_WHEELS], wheelContact[N_WHEELS];
    OControls ctrl;
    OInternal in;
    float brake, steer, drive;              /* staged, consumed next tick */
    float latF[N_WHEELS], lonF[N_WHEELS];   /* previous-tick wheel friction */
    int manCount;
    V3 manNormal;
    /* transient workspace of one tick */
    float brakePrev, steerPrev, drivePrev, throttleVal, rawThrottle, handbrakeVal;
    V3 jumpImp, angImp;
    float rayDist[N_WHEELS];
    V3 rayNormal[N_WHEELS];
    int cellIdx, numTris;
    int hitCount;
    OHit hits[MAX_TRI_PAIRS];
    int conCount[MAX_TRI_PAIRS];
    OContact contacts[MAX_TRI_PAIRS][MAX_PAIR_CONTACTS];
} OCar;

typedef struct {
    V3 pos, vel, ang, imp, intPos, intVel, expPos, expVel;
    int intValid;
    int blue, orange, lastScorer, goalTick, overtime;
    int episodeTicks, lastTouch, ballArenaContactTick;
    float pads[N_PADS];
} OSim;

typedef struct {
    int nVerts, nTris;
    V3* verts;
    int* tris;        /* 3 per triangle */
    V3* norms;
    V3* aabbMin;
    V3* aabbMax;
    V3* angs;         /* signed edge angle per triangle edge slot */
    int* cellTris;    /* per-cell triangle lists, ascending */
    int cellPrefix[N_CELLS + 1];
    /* native mesh metadata (CARL_ARENA_METADATA), else native == 0 and the
     * arrays are NULL: per triangle the order key (mesh * 10000 + order),
     * mesh, edge flags, three vertices in Bullet units, three edge angles */
    int native;
    int* nkey;
    int* nmesh;
    int* nflags;
    V3* nverts;
    V3* nangs;
    int* ballTris;    /* per-cell lists again, sorted by (order key, triangle) */
} OArena;

typedef struct {
    int nSim, nBlue, nOrange, nCars, nTotal, seed;
    int tickCount;
    OArena* arena;
    OCar* cars;
    OSim* sims;
} OWorld;

/* ---- shared helpers ---- */
O_INLINE V3 susp_connection(int w)
{
    const float x = w < 2 ? K_FRONT_SUSP_X : K_BACK_SUSP_X;
    const float ay = w < 2 ? K_FRONT_SUSP_Y : K_BACK_SUSP_Y;
    return v3(x, (w & 1) ? -ay : ay, 0.f);
}
O_INLINE float susp_ray_len(int w) { return w < 2 ? K_FRONT_RAY_LEN : K_BACK_RAY_LEN; }
O_INLINE float susp_radius(int w) { return w < 2 ? K_FRONT_WHEEL_RADIUS : K_BACK_WHEEL_RADIUS; }
O_INLINE float susp_rest(int w) { return w < 2 ? K_FRONT_SUSP_REST : K_BACK_SUSP_REST; }
O_INLINE float susp_scale(int w) { return w < 2 ? K_SUSP_SCALE_FRONT : K_SUSP_SCALE_BACK; }

/* arena.c */
OArena* oarena_load(const char* path, char* err, int errLen);
int oarena_load_metadata(OArena* a, const char* path, char* err, int errLen);
void oarena_free(OArena* a);
void oarena_cell3(V3 p, int* cx, int* cy, int* cz);
int oarena_flat(int cx, int cy, int cz);

/* physics.c */
void ophys_tick(OWorld* w, int kind, const void* actions);
void ophys_reset_all(OWorld* w);
void ophys_reset_to_kickoff(OWorld* w, int sim);
void ophys_reset_after_done(OWorld* w, int sim, int maxTicks, int overtimeTicks, int noTouchTicks);
void ophys_broadphase(OWorld* w, int car);
void ophys_raycast(OWorld* w, int car);
void ophys_init_empty_wheels(OCar* c, V3 up);
Q4 ophys_integrate_quat(Q4 rot, V3 ang);
void ophys_controls_decode(int kind, const void* actions, int car, OControls* out);
int ophys_kickoff_perm(int idx, int slot);
void ophys_probe_box_tri_sat(const float* tri, int* overlap, int* axisIdx, float* depth, float* axis);
int ophys_probe_box_tri_contacts(const float* tri, int* axisIdx, float* carPos, float* arenaPos, float* normal,
                                 float* depth);
int ophys_probe_manifold(OWorld* w, int ci, float* carPos, float* worldPos, float* normal, float* dist);
int ophys_probe_box_box_contacts(const float* cenA, const float* rotA, const float* cenB, const float* rotB,
                                 int* axisIdx, float* carPosA, float* carPosB, float* normal, float* depth);
void ophys_probe_box_box_sat(const float* cenA, const float* rotA, const float* cenB, const float* rotB,
                             int* overlap, int* axisIdx, float* depth);
V3 ophys_pad_pos(int pad);
int ophys_ball_hit_prev_tick(int hitTick, int tick);
int ophys_probe_ball_contacts(const OWorld* w, const float* center, int* tri, float* point, float* normal,
                              float* depth, float* reduction);

/* unit probes of reference behaviours (used by the known-answer tests) */
void ophys_probe_dodge(float pitch, float yaw, float roll, int* hasFlipped,
                       int* hasDoubleJumped, float* vel);
void ophys_probe_autoflip(const float* quat, int jump, int contacts, const float* normal,
                          int* isAutoFlipping, float* timer, float* ang);
float ophys_probe_ball_floor_split(float depth, float velz, int ballWasHit);
void ophys_probe_steer_stage(float staged, float* prevOut, float* curOut);

#endif
