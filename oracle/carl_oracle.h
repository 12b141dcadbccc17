/*
 * carl_oracle.h - C API of the CPU oracle (ctypes-friendly).
 *
 * TEST INFRASTRUCTURE (see omath.h): a sequential CPU restatement of the CARL
 * environment used to check the HIP engine.  The calls mirror the sequencing
 * of the reference binding (python/carl.cu EnvWrapper) over the reference
 * physics (include/Physics, include/State, src/Kernels.cu) and packing
 * (src/EnvIO.cu, include/Physics/Observations.cuh).  State export/import uses
 * the layout declared in include/carl_amd.h.
 */
#ifndef CARL_ORACLE_H
#define CARL_ORACLE_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef struct OEnv OEnv;

OEnv* oracle_create(int n_sim, int n_blue, int n_orange, int seed, int frameskip,
                    int flags, const char* obj_path, char* err, int err_len);
void oracle_destroy(OEnv* e);

/* EnvWrapper-level calls (python/carl.cu:286-706) */
void oracle_step(OEnv* e, int kind, const void* actions);
void oracle_reset(OEnv* e);
void oracle_set_ball(OEnv* e, const float* pos, const float* vel, const float* ang,
                     const int64_t* idx, int n_sel);
void oracle_set_car(OEnv* e, const float* pos, const float* rot, const float* vel,
                    const float* ang, const void* demoed, int demoed_is_byte,
                    const float* boost, const float* internal, const int64_t* idx,
                    int n_sel);
void oracle_apply_reset(OEnv* e, const float* bpos, const float* bvel, const float* bang,
                        const float* cpos, const float* crot, const float* cvel,
                        const float* cang, const void* demoed, int demoed_is_byte,
                        const float* boost, const float* internal, const int32_t* blue,
                        const int32_t* orange, const int32_t* ticks, const int64_t* idx,
                        int n_sel, const uint8_t* mask);
void oracle_set_match(OEnv* e, const int32_t* blue, const int32_t* orange,
                      const int32_t* ticks, const int64_t* idx, int n_sel);
void oracle_reset_pads(OEnv* e, const int64_t* idx, int n_sel);

/* lower-level calls */
void oracle_tick(OEnv* e, int kind, const void* actions, int n_ticks);
void oracle_reset_dones(OEnv* e);
int oracle_set_param(OEnv* e, int param, int value);
int oracle_get_param(OEnv* e, int param);

/* outputs: same ids, shapes and dtypes as carl_env_buffer; returns element count */
long oracle_buffer(OEnv* e, int id, void** data);

/* state checkpoint in the carl_amd.h layout */
void oracle_export(OEnv* e, uint32_t* car_state, uint32_t* sim_state, int* tick);
void oracle_import(OEnv* e, const uint32_t* car_state, const uint32_t* sim_state, int tick);

/* arena inspection (for broadphase / grid checks) */
int oracle_arena_counts(OEnv* e, int* n_verts, int* n_tris, int* n_refs);
void oracle_arena_copy(OEnv* e, float* verts, int32_t* tris, float* angles,
                       int32_t* cell_prefix, int32_t* cell_tris);
void oracle_cell_of(float x, float y, float z, int* cell3);
/* broadphase cell + candidate count of every car for the current state */
void oracle_broadphase(OEnv* e, int32_t* cell, int32_t* count);
/* suspension raycast of every car: dist [n,4], normal [n,4,3], source [n,4] */
void oracle_raycast(OEnv* e, float* dist, float* normal, int32_t* source);
/* ball-arena contacts for a ball centred at `center` (at most 68): triangle,
 * point [3], normal [3], depth, reduction offset [3]; returns the count */
int oracle_ball_contacts(OEnv* e, const float* center, int32_t* tri, float* point, float* normal,
                         float* depth, float* reduction);

/* known-answer probes (tests/physics_regressions.cu, tests/turtle_recovery.cu) */
int oracle_ball_hit_prev_tick(int hit_tick, int tick);
float oracle_probe_ball_floor_split(float depth, float velz, int ball_was_hit);
void oracle_probe_dodge(float pitch, float yaw, float roll, int* has_flipped,
                        int* has_double_jumped, float* vel);
void oracle_probe_autoflip(const float* quat, int jump, int contacts, const float* normal,
                           int* is_auto_flipping, float* timer, float* ang);
void oracle_probe_steer_stage(float staged, float* prev_out, float* cur_out);
int oracle_kickoff_perm(int idx, int slot);
/* SAT probes: triangle in box-local coordinates; two car hitboxes in world */
void oracle_probe_box_tri_sat(const float* tri, int* overlap, int* axis_idx, float* depth, float* axis);
int oracle_probe_box_tri_contacts(const float* tri, int* axis_idx, float* car_pos, float* arena_pos, float* normal,
                                  float* depth);
/* arena manifold of one car from the environment's current state */
int oracle_probe_manifold(OEnv* env, int car, float* car_pos, float* world_pos, float* normal, float* dist);
int oracle_probe_box_box_contacts(const float* cen_a, const float* rot_a, const float* cen_b, const float* rot_b,
                                  int* axis_idx, float* car_pos_a, float* car_pos_b, float* normal, float* depth);
void oracle_probe_box_box_sat(const float* cen_a, const float* rot_a, const float* cen_b, const float* rot_b,
                              int* overlap, int* axis_idx, float* depth);
uint32_t oracle_hash32(uint32_t v);
void oracle_sincos(float x, float* s, float* c);
float oracle_atan2(float y, float x);
void oracle_integrate_quat(const float* rot, const float* ang, float* out);

/* multi-threaded CPU throughput run: one arena (1v1) per thread, seeded
 * direct controls resampled every 8 ticks; returns total sim-ticks/s. */
double oracle_cpu_throughput(const char* obj_path, int threads, int ticks_per_thread,
                             int seed);

#ifdef __cplusplus
}
#endif

#endif
