/*
 * omath.h - scalar / vector / quaternion arithmetic of the CPU oracle.
 *
 * TEST INFRASTRUCTURE.  This directory is the CPU restatement of the CARL
 * reference used only as a checker (tests/, __graft_entry__.smoke() and the
 * cpu_baseline leg of bench.py).  The product never links it.
 *
 * Evaluation-order contract.  Every expression is written in the operand order
 * of the reference (include/Cuda/Math.cuh), compiled without floating-point
 * contraction, so each +,-,*,/,sqrt is one IEEE-754 binary32 operation.  The
 * only non-basic functions are:
 *   - o_sincos / o_atan2: own implementations of the Cephes single precision
 *     sinf/cosf/atanf method (S. L. Moshier, Cephes Math Library 2.2:
 *     Cody-Waite reduction by pi/2 and minimax polynomials on [-pi/4, pi/4];
 *     atan via the tan(pi/8) / tan(3pi/8) argument reduction), used in place
 *     of the reference's sinf/cosf/__sincosf/atan2f;
 *   - o_rsqrt(x) = 1/sqrt(x), used in place of the reference's rsqrtf;
 *   - o_min / o_max as plain comparisons (fminf/fmaxf differ only in the sign
 *     of an equal zero, which the comparison form pins).
 * The HIP engine follows the same contract, which is what lets a simulation
 * tick agree bit for bit between the two.
 *
 * Pinned by the reference's own known-answer tests, its tables, closed forms,
 * linear-programming SAT checks, brute-force mesh searches and physics laws
 * (momentum, restitution, Coulomb friction, spring equilibrium, rolling) on
 * isolated contacts, the game's published control numbers (jump, dodge, flip,
 * air control, drive and brake, steering radius, autoroll) and brute-force
 * contact geometry (clip polygons, edge closest points, support corners, the
 * kept manifold contact, seam normals at coplanar and angled mesh edges), the
 * handbrake's rise and fall, the powerslide steer blend measured from the
 * front axle's impulse direction, and the wheels' slip- and handbrake-scaled
 * friction (tests/).  Every function of the oracle has such a check.
 */
#ifndef CARL_ORACLE_MATH_H
#define CARL_ORACLE_MATH_H

#include <math.h>
#include <stdint.h>

typedef struct { float x, y, z; } V3;
typedef struct { float x, y, z, w; } Q4;

#define O_INLINE static inline

/* ---- scalars ---- */
O_INLINE float o_min(float a, float b) { return a < b ? a : b; }
O_INLINE float o_max(float a, float b) { return a > b ? a : b; }
/* reference clampf: fmaxf(lo, fminf(hi, v)) (Math.cuh:31-34) */
O_INLINE float o_clamp(float v, float lo, float hi) { return o_max(lo, o_min(hi, v)); }
O_INLINE float o_rsqrt(float x) { return 1.0f / sqrtf(x); }

static const float O_PI = 3.14159265358979323846f;

/* Cephes sinf/cosf: x = k*(pi/2) + r, |r| <= pi/4. */
O_INLINE void o_sincos(float x, float* s, float* c)
{
    const float twoOverPi = 0.636619772367581343f;
    const float p1 = 1.5703125f;                       /* pi/2 split, 8+ bits */
    const float p2 = 4.837512969970703125e-4f;
    const float p3 = 7.54978995489188216e-8f;
    const float kf = x * twoOverPi + (x >= 0.0f ? 0.5f : -0.5f);
    const int k = (int)kf;
    const float fk = (float)k;
    const float r = ((x - fk * p1) - fk * p2) - fk * p3;
    const float z = r * r;
    const float sp = ((-1.9515295891e-4f * z + 8.3321608736e-3f) * z - 1.6666654611e-1f) * z * r + r;
    const float cp = ((2.443315711809948e-5f * z - 1.388731625493765e-3f) * z + 4.166664568298827e-2f) * z * z
                   - 0.5f * z + 1.0f;
    switch (k & 3) {
    case 0: *s = sp; *c = cp; break;
    case 1: *s = cp; *c = -sp; break;
    case 2: *s = -sp; *c = -cp; break;
    default: *s = -cp; *c = sp; break;
    }
}
O_INLINE float o_sin(float x) { float s, c; o_sincos(x, &s, &c); return s; }
O_INLINE float o_cos(float x) { float s, c; o_sincos(x, &s, &c); return c; }

/* Cephes atanf */
O_INLINE float o_atan(float x)
{
    const float ax = x < 0.0f ? -x : x;
    float y, t;
    if (ax > 2.414213562373095f) { y = 1.5707963267948966f; t = -1.0f / ax; }
    else if (ax > 0.4142135623730950f) { y = 0.7853981633974483f; t = (ax - 1.0f) / (ax + 1.0f); }
    else { y = 0.0f; t = ax; }
    const float z = t * t;
    y = y + (((8.05374449538e-2f * z - 1.38776856032e-1f) * z + 1.99777106478e-1f) * z - 3.33329491539e-1f) * z * t + t;
    return x < 0.0f ? -y : y;
}

O_INLINE float o_atan2(float y, float x)
{
    if (x == 0.0f) {
        if (y > 0.0f) return 1.5707963267948966f;
        if (y < 0.0f) return -1.5707963267948966f;
        return 0.0f;
    }
    if (y == 0.0f) return x < 0.0f ? O_PI : 0.0f;
    const float w = x < 0.0f ? (y < 0.0f ? -O_PI : O_PI) : 0.0f;
    return w + o_atan(y / x);
}

/* ---- vectors (Math.cuh:36-190) ---- */
O_INLINE V3 v3(float x, float y, float z) { V3 r = { x, y, z }; return r; }
O_INLINE V3 vadd(V3 a, V3 b) { return v3(a.x + b.x, a.y + b.y, a.z + b.z); }
O_INLINE V3 vsub(V3 a, V3 b) { return v3(a.x - b.x, a.y - b.y, a.z - b.z); }
O_INLINE V3 vmul(V3 a, V3 b) { return v3(a.x * b.x, a.y * b.y, a.z * b.z); }
O_INLINE V3 vdiv(V3 a, V3 b) { return v3(a.x / b.x, a.y / b.y, a.z / b.z); }
O_INLINE V3 vadds(V3 a, float s) { return v3(a.x + s, a.y + s, a.z + s); }
O_INLINE V3 vsubs(V3 a, float s) { return v3(a.x - s, a.y - s, a.z - s); }
O_INLINE V3 vscale(V3 a, float s) { return v3(a.x * s, a.y * s, a.z * s); }
O_INLINE V3 vdivs(V3 a, float s) { return v3(a.x / s, a.y / s, a.z / s); }
O_INLINE V3 vneg(V3 a) { return v3(-a.x, -a.y, -a.z); }
O_INLINE V3 vabs(V3 a) { return v3(fabsf(a.x), fabsf(a.y), fabsf(a.z)); }
O_INLINE V3 vsign(V3 a) { return v3(a.x >= 0.f ? 1.f : -1.f, a.y >= 0.f ? 1.f : -1.f, a.z >= 0.f ? 1.f : -1.f); }
O_INLINE float vdot(V3 a, V3 b) { return a.x * b.x + a.y * b.y + a.z * b.z; }
O_INLINE V3 vcross(V3 a, V3 b) { return v3(a.y * b.z - a.z * b.y, a.z * b.x - a.x * b.z, a.x * b.y - a.y * b.x); }
O_INLINE float vlensq(V3 a) { return vdot(a, a); }
O_INLINE float vlen(V3 a) { return sqrtf(vlensq(a)); }
O_INLINE V3 vnorm(V3 a) { return vdivs(a, vlen(a)); }
O_INLINE V3 vmin(V3 a, V3 b) { return v3(o_min(a.x, b.x), o_min(a.y, b.y), o_min(a.z, b.z)); }
O_INLINE V3 vmax(V3 a, V3 b) { return v3(o_max(a.x, b.x), o_max(a.y, b.y), o_max(a.z, b.z)); }
O_INLINE float vget(V3 a, int i) { return i == 0 ? a.x : (i == 1 ? a.y : a.z); }
O_INLINE void vset(V3* a, int i, float v) { if (i == 0) a->x = v; else if (i == 1) a->y = v; else a->z = v; }
O_INLINE int vargmax(V3 a) { return a.y > a.x ? (a.y > a.z ? 1 : 2) : (a.x > a.z ? 0 : 2); }
O_INLINE int vgte(V3 a, float s) { return a.x >= s && a.y >= s && a.z >= s; }
static const V3 V_ZERO = { 0.f, 0.f, 0.f };
static const V3 V_X = { 1.f, 0.f, 0.f };
static const V3 V_Y = { 0.f, 1.f, 0.f };
static const V3 V_Z = { 0.f, 0.f, 1.f };
O_INLINE V3 v_axis(int i) { return i == 0 ? V_X : (i == 1 ? V_Y : V_Z); }

/* ---- quaternions, xyzw (Math.cuh:233-331) ---- */
O_INLINE Q4 q4(float x, float y, float z, float w) { Q4 q = { x, y, z, w }; return q; }
O_INLINE Q4 qscale(Q4 q, float s) { return q4(q.x * s, q.y * s, q.z * s, q.w * s); }
O_INLINE float qdot(Q4 a, Q4 b) { return (a.x * b.x + a.z * b.z) + (a.y * b.y + a.w * b.w); }
O_INLINE float qlensq(Q4 q) { return qdot(q, q); }
O_INLINE float qlen(Q4 q) { return sqrtf(qlensq(q)); }
O_INLINE Q4 qnormalize(Q4 q) { return qscale(q, 1.f / qlen(q)); }
O_INLINE Q4 qconj(Q4 q) { return q4(-q.x, -q.y, -q.z, q.w); }
O_INLINE Q4 qcomp(Q4 a, Q4 q)
{
    return q4((a.w * q.x - a.z * q.y) + (a.x * q.w + a.y * q.z),
              (a.w * q.y - a.x * q.z) + (a.y * q.w + a.z * q.x),
              (a.w * q.z - a.y * q.x) + (a.z * q.w + a.x * q.y),
              (a.w * q.w - a.z * q.z) - (a.x * q.x + a.y * q.y));
}
O_INLINE V3 qworld(Q4 q, V3 v)
{
    const V3 u = v3(q.x, q.y, q.z);
    const V3 t = vscale(vcross(u, v), 2.f / qlensq(q));
    return vadd(vadd(v, vscale(t, q.w)), vcross(u, t));
}
O_INLINE V3 qlocal(Q4 q, V3 v) { return qworld(qconj(q), v); }
O_INLINE Q4 qangle(float a)
{
    float s, c;
    o_sincos(a / 2.f, &s, &c);
    return q4(0.f, 0.f, s, c);
}
/* rotation matrix columns -> quaternion (Math.cuh:252-274) */
O_INLINE Q4 qfromaxes(V3 f, V3 r, V3 u)
{
    const float trace = f.x + r.y + u.z;
    const V3 t = vadds(vscale(v3(f.x, r.y, u.z), 2.f), 1.f - trace);
    const V3 sum = v3(r.z + u.y, u.x + f.z, f.y + r.x);
    const V3 diff = v3(r.z - u.y, u.x - f.z, f.y - r.x);
    if (trace > 0.f) {
        const float tw = 1.f + trace;
        return qscale(q4(diff.x, diff.y, diff.z, tw), .5f / sqrtf(tw));
    }
    switch (vargmax(t)) {
    case 0: return qscale(q4(t.x, sum.z, sum.y, diff.x), .5f / sqrtf(t.x));
    case 1: return qscale(q4(sum.z, t.y, sum.x, diff.y), .5f / sqrtf(t.y));
    default: return qscale(q4(sum.y, sum.x, t.z, diff.z), .5f / sqrtf(t.z));
    }
}

/* ---- integer mixer (include/Cuda/Random.cuh:7-17) ---- */
O_INLINE uint32_t o_hash32(uint32_t v)
{
    v = ((v >> 16) ^ v) * 0x45d9f3bu;
    v = ((v >> 16) ^ v) * 0x45d9f3bu;
    return (v >> 16) ^ v;
}
O_INLINE int o_random_index(uint32_t seed, int count) { return (int)(o_hash32(seed) % (uint32_t)count); }

/* Rodrigues rotation (include/Arena/TriMesh.cuh:72-76) */
O_INLINE V3 o_rotate_axis(V3 v, V3 ax, float a)
{
    float s, c;
    o_sincos(a, &s, &c);
    return vadd(vadd(vscale(v, c), vscale(vcross(ax, v), s)), vscale(ax, vdot(ax, v) * (1.f - c)));
}

#endif
