// dmath.h - device arithmetic for the CARL step engine (gfx950).
//
// Evaluation-order contract: every expression keeps the operand order of the
// reference vector library (include/Cuda/Math.cuh) and the file is compiled
// with -ffp-contract=off, so each + - * / sqrt is one IEEE binary32 op.
// Transcendentals are this engine's own: sin/cos/atan follow the Cephes
// single-precision method (S. L. Moshier, Cephes Math Library 2.2:
// Cody-Waite reduction by pi/2 and minimax polynomials on [-pi/4, pi/4];
// atan with tan(pi/8) / tan(3pi/8) argument reduction), rsqrt is 1/sqrt and
// min/max are plain comparisons.  Results therefore do not depend on the
// device math library, and a CPU program following the same contract
// reproduces them bit for bit.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#define DI __device__ __forceinline__
#define HDI __host__ __device__ __forceinline__

namespace carl {

HDI float fmin_(float a, float b) { return a < b ? a : b; }
HDI float fmax_(float a, float b) { return a > b ? a : b; }
HDI float clamp_(float v, float lo, float hi) { return fmax_(lo, fmin_(hi, v)); }
HDI float rsqrt_(float x) { return 1.0f / sqrtf(x); }

constexpr float kPi = 3.14159265358979323846f;

HDI void sincos_(float x, float* s, float* c)
{
    constexpr float twoOverPi = 0.636619772367581343f;
    constexpr float p1 = 1.5703125f;
    constexpr float p2 = 4.837512969970703125e-4f;
    constexpr float p3 = 7.54978995489188216e-8f;
    const float kf = x * twoOverPi + (x >= 0.0f ? 0.5f : -0.5f);
    const int k = (int)kf;
    const float fk = (float)k;
    const float r = ((x - fk * p1) - fk * p2) - fk * p3;
    const float z = r * r;
    const float sp = ((-1.9515295891e-4f * z + 8.3321608736e-3f) * z - 1.6666654611e-1f) * z * r + r;
    const float cp = ((2.443315711809948e-5f * z - 1.388731625493765e-3f) * z + 4.166664568298827e-2f) * z * z
                   - 0.5f * z + 1.0f;
    const int q = k & 3;
    *s = q == 0 ? sp : (q == 1 ? cp : (q == 2 ? -sp : -cp));
    *c = q == 0 ? cp : (q == 1 ? -sp : (q == 2 ? -cp : sp));
}

HDI float atan_(float x)
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

HDI float atan2_(float y, float x)
{
    if (x == 0.0f) {
        if (y > 0.0f) return 1.5707963267948966f;
        if (y < 0.0f) return -1.5707963267948966f;
        return 0.0f;
    }
    if (y == 0.0f) return x < 0.0f ? kPi : 0.0f;
    const float w = x < 0.0f ? (y < 0.0f ? -kPi : kPi) : 0.0f;
    return w + atan_(y / x);
}

struct V3 {
    float x, y, z;
};

HDI V3 mk(float x, float y, float z) { return V3{ x, y, z }; }
HDI V3 operator+(V3 a, V3 b) { return V3{ a.x + b.x, a.y + b.y, a.z + b.z }; }
HDI V3 operator-(V3 a, V3 b) { return V3{ a.x - b.x, a.y - b.y, a.z - b.z }; }
HDI V3 operator*(V3 a, V3 b) { return V3{ a.x * b.x, a.y * b.y, a.z * b.z }; }
HDI V3 operator/(V3 a, V3 b) { return V3{ a.x / b.x, a.y / b.y, a.z / b.z }; }
HDI V3 operator*(V3 a, float s) { return V3{ a.x * s, a.y * s, a.z * s }; }
HDI V3 operator/(V3 a, float s) { return V3{ a.x / s, a.y / s, a.z / s }; }
HDI V3 operator+(V3 a, float s) { return V3{ a.x + s, a.y + s, a.z + s }; }
HDI V3 operator-(V3 a, float s) { return V3{ a.x - s, a.y - s, a.z - s }; }
HDI V3 operator-(V3 a) { return V3{ -a.x, -a.y, -a.z }; }
HDI V3 vabs(V3 a) { return V3{ fabsf(a.x), fabsf(a.y), fabsf(a.z) }; }
HDI float l1norm(V3 a) { return (fabsf(a.x) + fabsf(a.y)) + fabsf(a.z); }
HDI V3 vsign(V3 a) { return V3{ a.x >= 0.f ? 1.f : -1.f, a.y >= 0.f ? 1.f : -1.f, a.z >= 0.f ? 1.f : -1.f }; }
HDI float dot(V3 a, V3 b) { return a.x * b.x + a.y * b.y + a.z * b.z; }
HDI V3 cross(V3 a, V3 b) { return V3{ a.y * b.z - a.z * b.y, a.z * b.x - a.x * b.z, a.x * b.y - a.y * b.x }; }
HDI float lensq(V3 a) { return dot(a, a); }
HDI float len(V3 a) { return sqrtf(lensq(a)); }
HDI V3 normalize(V3 a) { return a / len(a); }
HDI V3 vmin(V3 a, V3 b) { return V3{ fmin_(a.x, b.x), fmin_(a.y, b.y), fmin_(a.z, b.z) }; }
HDI V3 vmax(V3 a, V3 b) { return V3{ fmax_(a.x, b.x), fmax_(a.y, b.y), fmax_(a.z, b.z) }; }
HDI float comp(V3 a, int i) { return i == 0 ? a.x : (i == 1 ? a.y : a.z); }
// Member-wise select: a plain ?: on an aggregate selects between the two
// addresses and copies through memory, which pins both into scratch.
HDI float sel(bool c, float a, float b) { return c ? a : b; }
HDI V3 sel(bool c, V3 a, V3 b) { return V3{ c ? a.x : b.x, c ? a.y : b.y, c ? a.z : b.z }; }

// a[idx] = v for a small register array: every slot is rewritten through a
// member-wise select, so no dynamic address is formed and the array stays in
// registers (a conditional store per slot can be merged into one indexed
// store, which forces the array into scratch memory).
template <typename T, int N>
HDI void setAt(T (&a)[N], int idx, const T& v)
{
#pragma unroll
    for (int j = 0; j < N; j++) a[j] = sel(j == idx, v, a[j]);
}

HDI void setComp(V3& a, int i, float v) { if (i == 0) a.x = v; else if (i == 1) a.y = v; else a.z = v; }
HDI int argmax3(V3 a) { return a.y > a.x ? (a.y > a.z ? 1 : 2) : (a.x > a.z ? 0 : 2); }
HDI V3 unitAxis(int i) { return V3{ i == 0 ? 1.f : 0.f, i == 1 ? 1.f : 0.f, i == 2 || (i != 0 && i != 1) ? 1.f : 0.f }; }
constexpr V3 kZero{ 0.f, 0.f, 0.f };
constexpr V3 kX{ 1.f, 0.f, 0.f };
constexpr V3 kY{ 0.f, 1.f, 0.f };
constexpr V3 kZ{ 0.f, 0.f, 1.f };

struct Q4 {
    float x, y, z, w;
};

HDI Q4 qscale(Q4 q, float s) { return Q4{ q.x * s, q.y * s, q.z * s, q.w * s }; }
HDI float qdot(Q4 a, Q4 b) { return (a.x * b.x + a.z * b.z) + (a.y * b.y + a.w * b.w); }
HDI Q4 qnormalize(Q4 q) { return qscale(q, 1.f / sqrtf(qdot(q, q))); }
HDI Q4 qconj(Q4 q) { return Q4{ -q.x, -q.y, -q.z, q.w }; }
HDI Q4 qmul(Q4 a, Q4 q)
{
    return Q4{ (a.w * q.x - a.z * q.y) + (a.x * q.w + a.y * q.z),
               (a.w * q.y - a.x * q.z) + (a.y * q.w + a.z * q.x),
               (a.w * q.z - a.y * q.x) + (a.z * q.w + a.x * q.y),
               (a.w * q.w - a.z * q.z) - (a.x * q.x + a.y * q.y) };
}
// rotate v by q (q need not be unit: the cross term is scaled by 2/|q|^2)
HDI V3 rotate(Q4 q, V3 v)
{
    const V3 u{ q.x, q.y, q.z };
    const V3 t = cross(u, v) * (2.f / qdot(q, q));
    return (v + t * q.w) + cross(u, t);
}
HDI V3 unrotate(Q4 q, V3 v) { return rotate(qconj(q), v); }
HDI Q4 yawQuat(float a)
{
    float s, c;
    sincos_(a / 2.f, &s, &c);
    return Q4{ 0.f, 0.f, s, c };
}
// rotation with columns f, r, u (Shepperd's branch on the largest diagonal term)
HDI Q4 quatFromColumns(V3 f, V3 r, V3 u)
{
    const float trace = f.x + r.y + u.z;
    const V3 t = V3{ f.x, r.y, u.z } * 2.f + (1.f - trace);
    const V3 sum{ r.z + u.y, u.x + f.z, f.y + r.x };
    const V3 diff{ r.z - u.y, u.x - f.z, f.y - r.x };
    if (trace > 0.f) {
        const float tw = 1.f + trace;
        return qscale(Q4{ diff.x, diff.y, diff.z, tw }, .5f / sqrtf(tw));
    }
    const int m = argmax3(t);
    if (m == 0) return qscale(Q4{ t.x, sum.z, sum.y, diff.x }, .5f / sqrtf(t.x));
    if (m == 1) return qscale(Q4{ sum.z, t.y, sum.x, diff.y }, .5f / sqrtf(t.y));
    return qscale(Q4{ sum.y, sum.x, t.z, diff.z }, .5f / sqrtf(t.z));
}

HDI uint32_t mix32(uint32_t v)
{
    v = ((v >> 16) ^ v) * 0x45d9f3bu;
    v = ((v >> 16) ^ v) * 0x45d9f3bu;
    return (v >> 16) ^ v;
}
HDI int pickIndex(uint32_t seed, int n) { return (int)(mix32(seed) % (uint32_t)n); }

// Rodrigues rotation of v about unit axis ax by angle a
HDI V3 rodrigues(V3 v, V3 ax, float a)
{
    float s, c;
    sincos_(a, &s, &c);
    return (v * c + cross(ax, v) * s) + ax * (dot(ax, v) * (1.f - c));
}

}  // namespace carl
