/*
 * carl_amd.h - C-ABI of the MI355X CARL step engine.
 *
 * Plain pointers, sizes and int status codes; no C++ or torch types cross this
 * boundary.  Every entry point returns CARL_OK (0) or a negative status; the
 * message of the last failure on the calling thread is carl_last_error().
 *
 * The entry points replace the native layer that the reference binds from
 * python/carl.cu (pybind11 `carl._carl.Env`), i.e. the RLEnvironment and
 * EnvIO classes:
 *   carl_env_create        <- EnvWrapper::EnvWrapper     python/carl.cu:286-310
 *                             RLEnvironment ctor         src/RLEnvironment.cu:40-82
 *                             EnvIO ctor                 src/EnvIO.cu:361-414
 *   carl_env_destroy       <- EnvWrapper::~EnvWrapper    python/carl.cu:312-318
 *   carl_env_step          <- EnvWrapper::step / stepContinuous
 *                                                        python/carl.cu:320-370
 *   carl_env_tick          <- RLEnvironment::step (3 overloads)
 *                                                        src/RLEnvironment.cu:166-211
 *   carl_env_reset         <- EnvWrapper::reset          python/carl.cu:372-382
 *   carl_env_reset_dones   <- RLEnvironment::resetDones  src/RLEnvironment.cu:213-219
 *   carl_env_set_ball      <- EnvWrapper::setBall        python/carl.cu:385-420
 *   carl_env_set_car       <- EnvWrapper::setCar         python/carl.cu:422-506
 *   carl_env_apply_reset   <- EnvWrapper::applyResetState python/carl.cu:508-666
 *   carl_env_set_match     <- EnvWrapper::setMatchState  python/carl.cu:668-690
 *   carl_env_reset_pads    <- EnvWrapper::resetBoostPads python/carl.cu:692-706
 *   carl_env_buffer        <- EnvIO::get*Tensor          src/EnvIO.cu:665-718
 *   carl_env_set_param     <- EnvWrapper::set{MaxTicks,...,Frameskip}
 *                                                        python/carl.cu:782-818
 *   carl_env_stream        <- RLEnvironment::getStream   include/RLEnvironment.cuh:61
 *   carl_env_synchronize   <- cudaStreamSynchronize calls python/carl.cu:419,505,663
 *   carl_env_pack_rewards_dones    <- EnvIO::packRewardsDones    src/EnvIO.cu:466-484
 *   carl_env_pack_transition_state <- EnvIO::packTransitionState src/EnvIO.cu:442-448
 *   carl_env_pack_transition_obs   <- EnvIO::packTransitionObs   src/EnvIO.cu:458-464
 *   carl_env_pack_match_state      <- EnvIO::packRawMatchState   src/EnvIO.cu:486-497
 *   carl_env_pack_obs              <- EnvIO::packObs             src/EnvIO.cu:450-456
 *   carl_env_pack_state            <- EnvIO::packState           src/EnvIO.cu:434-440
 *   carl_env_set_actions           <- EnvIO::setActions / setContinuousActions
 *                                                                src/EnvIO.cu:565-577
 *   carl_exclusive_scan_i32 <- PrefixSum::scanOnStream   src/RLEnvironment.cu:18-38
 *
 * carl_env_enable_timing / carl_env_tick_timing / carl_tick_kernel_name have no
 * reference counterpart: they time the tick kernels with HIP events on the
 * environment stream.
 * carl_env_export_state / carl_env_import_state have no reference counterpart;
 * they expose the persistent per-car / per-simulation state (layout below) so
 * that a CPU model can be stepped from the same state and compared field by
 * field, and so callers can checkpoint an environment.
 *
 * All device pointers must live on the device the environment was created on
 * (HIP device 0, matching the reference's hard-coded cuda:0).  Work is
 * enqueued on the environment's private stream and is asynchronous unless a
 * function says otherwise.
 */
#ifndef CARL_AMD_H
#define CARL_AMD_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- status codes ---------------------------------------------------- */
enum {
    CARL_OK = 0,
    CARL_ERR_VALUE = -1,   /* invalid argument value  (Python ValueError) */
    CARL_ERR_TYPE = -2,    /* invalid argument type   (Python TypeError)  */
    CARL_ERR_RUNTIME = -3, /* device / runtime failure                    */
    CARL_ERR_ARENA = -4    /* arena mesh missing or malformed             */
};

/* ---- creation flags -------------------------------------------------- */
enum {
    CARL_FLAG_INVERT_ORANGE = 1,
    CARL_FLAG_NORMALIZE = 2,
    CARL_FLAG_PREVIOUS_CONTROLS = 4
};

/* ---- action kinds ----------------------------------------------------- */
enum {
    CARL_ACTIONS_DISCRETE = 0,   /* int32 [n_sim, n_cars, 7], values 0/1/2      */
    CARL_ACTIONS_CONTINUOUS = 1, /* float [n_sim, n_cars, 7]                    */
    CARL_ACTIONS_DIRECT = 2      /* CarControls [n_sim*n_cars]: 5 f32 + 3 i32   */
};

/* ---- output buffers (carl_env_buffer ids) ----------------------------- */
enum {
    CARL_BUF_OBS = 0,                      /* f32  [n_sim, n_cars, obs_dim] */
    CARL_BUF_TRANSITION_OBS = 1,           /* f32  [n_sim, n_cars, obs_dim] */
    CARL_BUF_STATE = 2,                    /* f32  [n_sim, state_dim]       */
    CARL_BUF_TRANSITION_STATE = 3,         /* f32  [n_sim, state_dim]       */
    CARL_BUF_ACTIONS = 4,                  /* i32  [n_sim, n_cars, 7]       */
    CARL_BUF_REWARDS = 5,                  /* f32  [n_sim]                  */
    CARL_BUF_DONES = 6,                    /* bool [n_sim]                  */
    CARL_BUF_SCORE_DIFFERENCE = 7,         /* i32  [n_sim]                  */
    CARL_BUF_EPISODE_TICKS = 8,            /* i32  [n_sim]                  */
    CARL_BUF_TRANSITION_SCORE_DIFFERENCE = 9,
    CARL_BUF_TRANSITION_EPISODE_TICKS = 10,
    CARL_BUF_OVERTIME = 11,                /* bool [n_sim]                  */
    CARL_BUF_TRANSITION_OVERTIME = 12,
    CARL_BUF_CONTINUOUS_ACTIONS = 13,      /* f32  [n_sim, n_cars, 7]       */
    CARL_BUF_COUNT = 14
};

enum { CARL_DTYPE_F32 = 0, CARL_DTYPE_I32 = 1, CARL_DTYPE_BOOL = 2 };

/* ---- parameters (carl_env_set_param / carl_env_get_param) ------------- */
enum {
    CARL_PARAM_MAX_TICKS = 0,
    CARL_PARAM_OVERTIME_TIMEOUT_TICKS = 1,
    CARL_PARAM_NO_TOUCH_TIMEOUT_TICKS = 2,
    CARL_PARAM_FRAMESKIP = 3,
    CARL_PARAM_N_SIM = 4,        /* read-only */
    CARL_PARAM_N_CARS = 5,       /* read-only */
    CARL_PARAM_OBS_DIM = 6,      /* read-only */
    CARL_PARAM_ACT_DIM = 7,      /* read-only */
    CARL_PARAM_STATE_DIM = 8,    /* read-only */
    CARL_PARAM_TICK_COUNT = 9,   /* read-only: global physics tick counter */
    CARL_PARAM_N_BLUE = 10,      /* read-only */
    CARL_PARAM_TICK_STREAMS = 11, /* partitions of the simulations, each ticked on its own stream [1, 4];
                                     no reference counterpart (default 1) */
    CARL_PARAM_CONTACT_SCREEN = 12, /* 1: the contact search drops (car, triangle) pairs its float tests
                                      provably reject before running them; 0: it runs them on every pair.
                                      Results are identical; no reference counterpart (default 1) */
    CARL_PARAM_TICK_WINDOW = 13,   /* > 0: all ticks of a step in one launch per partition, this many
                                      simulations per workgroup (at most 128 cars; default 64, halved down
                                      to 8 for runs too small to fill the GPU until it is set); 0: four
                                      phase kernels per tick.  Results are identical; no reference
                                      counterpart */
    CARL_PARAM_NATIVE_ARENA = 14,  /* read-only: 1 when the environment was created with native mesh
                                      metadata (the reference's ArenaMesh::hasNativeMetadata) */
    CARL_PARAM_TICK_WINDOW_LAUNCH = 15, /* read-only: simulations per workgroup the next window launch
                                          uses (CARL_PARAM_TICK_WINDOW capped at 128 cars, after the
                                          automatic sizing of small runs; 0: phase kernels); no
                                          reference counterpart */
    CARL_PARAM_TICK_BALANCE = 16,  /* 1: 1v1 and 2v2 window launches of 64- and 32-simulation
                                      workgroups deal the simulations to the workgroups in units of
                                      32 cars (16 or 8 simulations), ordered by the contact work
                                      each unit did in the balanced launch before, so that the
                                      workgroups finish together; 0: workgroup b takes simulations
                                      [S b, S b + S).  Results are identical; no reference
                                      counterpart (default 1) */
    CARL_PARAM_TICK_BALANCED_LAUNCH = 17 /* read-only: 1 when the next step's window launch is
                                            dealt (1v1 or 2v2, one partition, workgroups of 64 or
                                            32 simulations, n_sim a multiple of that, mesh arena,
                                            frameskip at least 4, CARL_PARAM_TICK_BALANCE on); no
                                            reference counterpart */
};

/* ---- persistent state layout (export / import) ------------------------
 * Car state: CARL_CAR_FIELDS planes of n_sim*n_cars 32-bit words; plane f,
 * car c lives at word f*n_total_cars + c.  Simulation state: CARL_SIM_FIELDS
 * planes of n_sim words.  Fields marked (i) hold int32 bit patterns, the rest
 * IEEE float32.  Car c of simulation s is c = s*n_cars + local, blue cars
 * first.  These are exactly the quantities that survive from one physics
 * tick to the next (reference: include/State/GameState.cuh:9-232 plus the
 * cross-tick parts of include/State/Workspace.cuh:8-234).                */
enum {
    CARL_CAR_POS = 0,             /* x,y,z */
    CARL_CAR_VEL = 3,
    CARL_CAR_ANG = 6,
    CARL_CAR_ROT = 9,             /* quaternion x,y,z,w */
    CARL_CAR_CEN = 13,            /* hitbox centre x,y,z */
    CARL_CAR_IMP = 16,            /* cached bump impulse x,y,z */
    CARL_CAR_DEMOED = 19,         /* (i) */
    CARL_CAR_DEMO_TIMER = 20,
    CARL_CAR_CONTACT_IDX = 21,    /* (i) last bumped car */
    CARL_CAR_CONTACT_COOLDOWN = 22,
    CARL_CAR_BALL_HIT_TICK = 23,  /* (i) */
    CARL_CAR_BALL_CONTACT_TICK = 24, /* (i) */
    CARL_CAR_ARENA_CONTACT_TICK = 25, /* (i) */
    CARL_CAR_WHEEL_SOURCE = 26,   /* (i) x4 */
    CARL_CAR_WHEEL_CONTACT = 30,  /* (i) x4 */
    CARL_CAR_CTRL_THROTTLE = 34,
    CARL_CAR_CTRL_STEER = 35,
    CARL_CAR_CTRL_YAW = 36,
    CARL_CAR_CTRL_PITCH = 37,
    CARL_CAR_CTRL_ROLL = 38,
    CARL_CAR_CTRL_JUMP = 39,      /* (i) */
    CARL_CAR_CTRL_BOOST = 40,     /* (i) */
    CARL_CAR_CTRL_SLIDE = 41,     /* (i) */
    CARL_CAR_ON_GROUND = 42,      /* (i) */
    CARL_CAR_AIR_TIME = 43,
    CARL_CAR_AIR_TIME_SINCE_JUMP = 44,
    CARL_CAR_HANDBRAKE = 45,
    CARL_CAR_HAS_JUMPED = 46,     /* (i) */
    CARL_CAR_IS_JUMPING = 47,     /* (i) */
    CARL_CAR_JUMP_TIME = 48,
    CARL_CAR_LAST_JUMP = 49,      /* (i) */
    CARL_CAR_HAS_DOUBLE_JUMPED = 50, /* (i) */
    CARL_CAR_HAS_FLIPPED = 51,    /* (i) */
    CARL_CAR_IS_FLIPPING = 52,    /* (i) */
    CARL_CAR_FLIP_TIME = 53,
    CARL_CAR_IS_AUTO_FLIPPING = 54, /* (i) */
    CARL_CAR_AUTO_FLIP_TIMER = 55,
    CARL_CAR_AUTO_FLIP_SCALE = 56,
    CARL_CAR_FLIP_TORQUE = 57,    /* x,y,z */
    CARL_CAR_RESPAWN_IDX = 60,    /* (i) */
    CARL_CAR_LAST_RESPAWN_DIR = 61, /* (i) */
    CARL_CAR_IS_BOOSTING = 62,    /* (i) */
    CARL_CAR_BOOST = 63,
    CARL_CAR_BOOSTING_TIME = 64,
    CARL_CAR_TIME_SINCE_BOOSTED = 65,
    CARL_CAR_BRAKE_STAGE = 66,    /* staged brake factor, consumed next tick */
    CARL_CAR_STEER_STAGE = 67,    /* staged steer angle, consumed next tick  */
    CARL_CAR_DRIVE_STAGE = 68,    /* staged engine drive, consumed next tick */
    CARL_CAR_LAT_FRICTION = 69,   /* x4 wheel friction of the previous tick */
    CARL_CAR_LON_FRICTION = 73,   /* x4 */
    CARL_CAR_MANIFOLD_COUNT = 77, /* (i) arena manifold size of the previous tick */
    CARL_CAR_MANIFOLD_NORMAL = 78,/* x,y,z first manifold normal */
    CARL_CAR_FIELDS = 81
};

enum {
    CARL_SIM_BALL_POS = 0,
    CARL_SIM_BALL_VEL = 3,
    CARL_SIM_BALL_ANG = 6,
    CARL_SIM_BALL_IMP = 9,
    CARL_SIM_BALL_INT_POS = 12,   /* integration position (Bullet units) */
    CARL_SIM_BALL_INT_VEL = 15,
    CARL_SIM_BALL_EXP_POS = 18,   /* last exported position */
    CARL_SIM_BALL_EXP_VEL = 21,
    CARL_SIM_BALL_INT_VALID = 24, /* (i) */
    CARL_SIM_BLUE_SCORE = 25,     /* (i) */
    CARL_SIM_ORANGE_SCORE = 26,   /* (i) */
    CARL_SIM_LAST_SCORER = 27,    /* (i) */
    CARL_SIM_GOAL_TICK = 28,      /* (i) */
    CARL_SIM_OVERTIME = 29,       /* (i) */
    CARL_SIM_EPISODE_TICKS = 30,  /* (i) */
    CARL_SIM_LAST_TOUCH_TICK = 31,/* (i) */
    CARL_SIM_BALL_ARENA_CONTACT_TICK = 32, /* (i) */
    CARL_SIM_PAD_COOLDOWN = 33,   /* x34 */
    CARL_SIM_FIELDS = 67
};

/* Direct per-car controls (reference CarControls, include/State/Controls.cuh:7-12). */
typedef struct carl_controls {
    float throttle, steer, yaw, pitch, roll;
    int32_t jump, boost, slide;
} carl_controls;

typedef struct carl_env carl_env;

/* ---- lifecycle ---------------------------------------------------------- */

/* Loads the arena mesh (env CARL_ARENA_OBJ, else carl_amd/assets/arena.obj next
 * to the library), allocates device state, resets every simulation to a
 * kickoff and packs the initial outputs.  frameskip >= 1.
 * n_sim * (n_blue + n_orange) must be at most 6,628,032 cars: the state is
 * addressed with 32-bit byte offsets.  A larger size fails with
 * CARL_ERR_VALUE before any allocation.
 * The arena is built once per process for each mesh (and metadata) file, and
 * the environments on one device share one device copy of it, freed with the
 * last of them (the reference builds its host mesh once per process,
 * src/ArenaMesh.cu:17-28).
 * When the environment variable CARL_ARENA_METADATA is set, its file holds
 * RocketSim's native mesh metadata for every triangle (the text that
 * tools/arena_metadata.py writes: the triangle count, then per triangle
 * "mesh order angle0 angle1 angle2 flags v0x v0y v0z v1x v1y v1z v2x v2y v2z"
 * with the vertices in Bullet units, src/ArenaMesh.cu:69-99), and the ball
 * meets the arena as the native meshes do (BallArena/Contact.cuh:292-594).
 * A count other than the mesh's triangle count (an unreadable file reads as
 * count 0) fails with CARL_ERR_ARENA "CARL arena metadata triangle count
 * mismatch"; a file that ends early or holds a non-number fails with
 * "Invalid CARL arena metadata". */
int carl_env_create(int n_sim, int n_blue, int n_orange, int seed, int frameskip,
                    int flags, carl_env** out);
int carl_env_destroy(carl_env* env);

/* The environment's private HIP stream (hipStream_t). */
void* carl_env_stream(carl_env* env);
int carl_env_synchronize(carl_env* env);

/* ---- stepping ------------------------------------------------------------ */

/* One environment step: runs `frameskip` physics ticks on actions (device
 * pointer, layout per kind), then packs rewards/dones, the transition
 * state/obs, resets finished simulations, packs the current obs/state and
 * leaves a copy of the actions in the environment's action buffer
 * (python/carl.cu:320-370).  The work is queued on the environment stream;
 * `actions` must stay unchanged until it has run. */
int carl_env_step(carl_env* env, int kind, const void* actions);

/* Physics ticks only, no packing (RLEnvironment::step). */
int carl_env_tick(carl_env* env, int kind, const void* actions, int n_ticks);

/* Full reset of every simulation to a kickoff plus the initial packs. */
int carl_env_reset(carl_env* env);

/* Reset simulations whose episode ended (goal, timeouts, overtime expiry). */
int carl_env_reset_dones(carl_env* env);

/* ---- EnvIO packs (for C++ hosts composing the step themselves) ----------
 * The step's post-tick sequence of python/carl.cu:359-367 is
 *   pack_rewards_dones; pack_transition_state(frameskip);
 *   pack_transition_obs; reset_dones; pack_match_state(NULL); pack_obs(NULL);
 *   pack_state(NULL)
 * and carl_env_step runs exactly that (fused) after its ticks.  reset_mask
 * (bool [n_sim], device) restricts a pack to the selected simulations; NULL
 * packs every simulation.  All are queued on the environment stream. */
int carl_env_pack_rewards_dones(carl_env* env);
int carl_env_pack_transition_state(carl_env* env, int touch_window);
int carl_env_pack_transition_obs(carl_env* env);   /* rows of the simulations whose done flag is set */
int carl_env_pack_match_state(carl_env* env, const uint8_t* reset_mask);
int carl_env_pack_obs(carl_env* env, const uint8_t* reset_mask);
int carl_env_pack_state(carl_env* env, const uint8_t* reset_mask);
/* Copy a step's actions (device pointer, CARL_ACTIONS_DISCRETE int32 or
 * CARL_ACTIONS_CONTINUOUS float [n_sim, n_cars, 7]) into the environment's
 * action buffer (CARL_BUF_ACTIONS / CARL_BUF_CONTINUOUS_ACTIONS). */
int carl_env_set_actions(carl_env* env, int kind, const void* actions);

/* ---- state setters --------------------------------------------------------
 * Row r of each input belongs to simulation indices[r] (int64, device) when
 * indices != NULL, else to simulation r.  With a mask (bool [n_sim], device)
 * row r is applied only where mask[r] is true and n_selected must be n_sim.
 * indices and mask are mutually exclusive.  Shapes: vectors [n_sel,3] or
 * [n_sel,n_cars,3], rotations [n_sel,n_cars,4] quaternion xyzw, demoed
 * [n_sel,n_cars] int32 or bool (demoed_is_byte), boost [n_sel,n_cars],
 * internal [n_sel,n_cars,19], scores/ticks [n_sel] int32.  Optional inputs
 * may be NULL. */
int carl_env_set_ball(carl_env* env, const float* pos, const float* vel,
                      const float* ang, const int64_t* indices, int n_selected);
int carl_env_set_car(carl_env* env, const float* pos, const float* rot,
                     const float* vel, const float* ang, const void* demoed,
                     int demoed_is_byte, const float* boost, const float* internal,
                     const int64_t* indices, int n_selected);
int carl_env_apply_reset(carl_env* env, const float* ball_pos, const float* ball_vel,
                         const float* ball_ang, const float* car_pos,
                         const float* car_rot, const float* car_vel,
                         const float* car_ang, const void* car_demoed,
                         int demoed_is_byte, const float* car_boost,
                         const float* car_internal, const int32_t* blue_score,
                         const int32_t* orange_score, const int32_t* episode_ticks,
                         const int64_t* indices, int n_selected,
                         const uint8_t* mask);
int carl_env_set_match(carl_env* env, const int32_t* blue_score,
                       const int32_t* orange_score, const int32_t* episode_ticks,
                       const int64_t* indices, int n_selected);
int carl_env_reset_pads(carl_env* env, const int64_t* indices, int n_selected);

/* ---- outputs and parameters --------------------------------------------- */

/* Device pointer, shape (up to 3 dims) and dtype of an output buffer.  The
 * memory belongs to the environment and is rewritten by later calls. */
int carl_env_buffer(carl_env* env, int id, void** data, int64_t* shape, int* ndim,
                    int* dtype);
int carl_env_set_param(carl_env* env, int param, int value);
int carl_env_get_param(carl_env* env, int param, int* value);

/* ---- state checkpoint (no reference counterpart) -------------------------
 * Host buffers of CARL_CAR_FIELDS*n_sim*n_cars and CARL_SIM_FIELDS*n_sim
 * 32-bit words.  Both synchronise the stream.  Import also sets the global
 * tick counter. */
int carl_env_export_state(carl_env* env, uint32_t* car_state, uint32_t* sim_state,
                          int* tick_count);
int carl_env_import_state(carl_env* env, const uint32_t* car_state,
                          const uint32_t* sim_state, int tick_count);

/* ---- tick-kernel timing (no reference counterpart) -------------------------
 * One physics tick is four phases, in this order (the reference's eleven
 * per-tick launches, src/RLEnvironment.cu:166-211, grouped by the data they
 * own): four kernels per tick, or one tick-window kernel running every phase
 * of every tick of a step (CARL_PARAM_TICK_WINDOW). */
enum {
    CARL_KERNEL_CONTACT = 0,    /* broadphase, wheel rays, car-arena contact search */
    CARL_KERNEL_CAR_ARENA = 1,  /* controls, suspension, car-arena solve */
    CARL_KERNEL_BALL = 2,       /* episode clock, car-car pairs, ball-arena, car-ball, goal */
    CARL_KERNEL_FINISH = 3,     /* integration, impulse caches, boost pads */
    CARL_KERNEL_WINDOW = 4,     /* all four phases of every tick of an env step, one launch */
    CARL_KERNEL_STEP_ENV = 5,   /* an env step's packing after its ticks (rewards/dones .. state) */
    CARL_TICK_KERNELS = 6
};

/* Timing selection for carl_env_enable_timing (bit flags; 0 turns it off). */
enum { CARL_TIME_TICKS = 1, CARL_TIME_PACKING = 2, CARL_TIME_STAGES = 4 };

/* With timing enabled, HIP events recorded by the dispatch bracket every
 * tick kernel of partition 0 (CARL_TIME_TICKS or CARL_TIME_STAGES) and every
 * packing kernel of carl_env_step (CARL_TIME_PACKING).  At most 1024 launches'
 * events are held; the 1025th launch first synchronises the environment
 * stream and adds their durations to the sums.
 * carl_env_tick_timing synchronises the environment stream and
 * returns, per kernel (arrays of CARL_TICK_KERNELS), the summed duration in
 * ms and the launch count since timing was enabled or last read, then clears
 * them.  Enabling or disabling also clears them. */
int carl_env_enable_timing(carl_env* env, int enable);
int carl_env_tick_timing(carl_env* env, double* kernel_ms, int* launches);
const char* carl_tick_kernel_name(int kernel);

/* ---- stage profile (the reference's PROFILE stages,
 * include/Cuda/Profiler.cuh:119-162, src/RLEnvironment.cu:166-211) ----------
 * The phases of a tick.  The reference's nine stages fall into them as:
 * contact = broad+susp, narrow; car-arena = controls, manifold+solve;
 * ball = car-car+ball; finish = integrate-cars, impulse-cache;
 * boost-pads = boost-pads. */
enum {
    CARL_STAGE_CONTACT = 0,
    CARL_STAGE_CAR_ARENA = 1,
    CARL_STAGE_BALL = 2,
    CARL_STAGE_FINISH = 3,
    CARL_STAGE_PADS = 4,
    CARL_STAGES = 5
};

/* With CARL_TIME_STAGES enabled, the tick window launches of partition 0 run
 * a twin of the window kernel in which each workgroup reads the device's
 * constant-rate wall clock at its start and at every phase barrier (the plain
 * kernel is left as it is: it is the one measured otherwise).
 * carl_env_stage_timing synchronises and returns, for the ticks since the
 * profile was enabled or last read, in us per tick:
 *   stage_us[CARL_STAGES]  each stage's share of the device: the stage's time
 *       summed over all workgroups / the workgroups resident at once
 *       (min(grid, occupancy x CUs)).  Workgroups that finish early leave
 *       their slots idle until the launch ends, so these sum to less than
 *       the launch time by the launch's imbalance.
 *   last_us[CARL_STAGES + 1]  the critical path: the stages of the workgroup
 *       that finished each launch last, then its start after the launch's
 *       first workgroup start; they sum to span_us.
 *   span_us    the launch's first workgroup start to its last workgroup end
 *       (wall clock).
 *   launch_us  the launch itself (HIP events).
 *   ticks      ticks covered;
 * then clears them.  With the phase kernels each stage is one kernel's
 * HIP-event time (the boost pads run in the finish kernel: CARL_STAGE_PADS
 * is 0), in stage_us and last_us alike, and span_us = launch_us = their sum.
 * It fails with CARL_ERR_VALUE when the profile is off or the tick launch
 * shape (window size, streams, window/phase path) changed within the period.
 * With several tick streams only partition 0 is profiled and the figures are
 * its own; the other partitions share the device. */
int carl_env_stage_timing(carl_env* env, double* stage_us, double* last_us, double* span_us,
                          double* launch_us, int* ticks);
const char* carl_stage_name(int stage);

/* ---- primitives ------------------------------------------------------------ */

/* Exclusive prefix sum of n int32 on a stream (device pointers; in == out
 * allowed).  Wave64 DPP/ballot scan, no library calls. */
int carl_exclusive_scan_i32(const int32_t* in, int32_t* out, int n, void* stream);

/* carl_exclusive_scan_i32 without any allocation: no counterpart in the
 * reference.  For callers that cannot allocate device memory (code under HIP
 * graph capture, tight serving loops, harnesses that forbid hipMalloc).  The
 * tile sums live in a fixed device array of 65,568 words (256 KiB) held by
 * each GPU the library runs on until the process ends; n may be at most
 * 67,108,864 (2^26), larger n returns CARL_ERR_VALUE.  The array belongs to
 * the device current at the call and is shared by every call on that GPU:
 * calls that overlap on one GPU (other streams, other threads) race.  Same
 * results as carl_exclusive_scan_i32. */
int carl_exclusive_scan_i32_noalloc(const int32_t* in, int32_t* out, int n, void* stream);

/* Message of the last failed call on this thread ("" if none). */
const char* carl_last_error(void);

/* Observation / state widths (reference include/Cuda/DLPack.h:95-107). */
int carl_observation_dim(int n_cars, int previous_controls);
int carl_state_dim(int n_cars);

#ifdef __cplusplus
}
#endif

#endif /* CARL_AMD_H */
