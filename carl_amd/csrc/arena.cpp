// arena.cpp - host construction of the soccar collision mesh and its
// LDS-stageable device layout.
//
// Semantics follow the reference mesh build:
//   OBJ "v" lines store (y, x, z); "f" lines are 1-based triangles
//                                       include/Arena/ObjLoader.cuh:91-126
//   vertices welded on exact bit equality (-0 == +0), first occurrence wins
//                                       include/Arena/ObjLoader.cuh:49-89
//   unit face normals, degenerate triangles rejected
//                                       include/Arena/TriMesh.cuh:26-44
//   triangle registered in grid cells [cell(aabbMin) - 1, cell(aabbMax)]
//                                       include/Arena/BroadPhaseGrid.cuh:30-78
//   signed dihedral angle per shared edge, 2*pi on boundary edges
//                                       include/Arena/EdgeInfo.cuh:60-125
#include "arena.h"

#include <algorithm>
#include <array>
#include <cmath>
#include <cstdlib>
#include <cstring>
#include <fstream>
#include <sstream>
#include <unordered_map>

#include "constants.h"
#include "state.h"

namespace carl {
namespace {

uint32_t keyBits(float v)
{
    if (v == 0.f) v = 0.f;
    uint32_t u;
    std::memcpy(&u, &v, 4);
    return u;
}

struct KeyHash {
    size_t operator()(const std::array<uint32_t, 3>& k) const
    {
        return (size_t)mix32(k[0] ^ mix32(k[1] ^ mix32(k[2])));
    }
};

}  // namespace

std::string findArenaObj(const std::string& libraryDir)
{
    if (const char* env = std::getenv("CARL_ARENA_OBJ")) {
        if (*env) return env;
    }
    const std::string candidates[] = { libraryDir + "/assets/arena.obj", libraryDir + "/../assets/arena.obj",
                                       "carl_amd/assets/arena.obj", "assets/arena.obj" };
    for (const auto& c : candidates) {
        std::ifstream f(c);
        if (f.is_open()) return c;
    }
    return libraryDir + "/assets/arena.obj";
}

std::string buildArena(const std::string& objPath, HostArena& out)
{
    std::ifstream file(objPath);
    if (!file.is_open()) return "failed to open assets/arena.obj";

    std::vector<V3> raw;
    std::vector<int> tris;
    std::string line;
    while (std::getline(file, line)) {
        std::istringstream s(line);
        std::string type;
        if (!(s >> type)) continue;
        if (type == "v") {
            std::string a, b, c;
            if (!(s >> a >> b >> c)) return "invalid OBJ vertex";
            // horizontal axes are swapped in the source file
            raw.push_back(V3{ std::strtof(b.c_str(), nullptr), std::strtof(a.c_str(), nullptr),
                              std::strtof(c.c_str(), nullptr) });
        } else if (type == "f") {
            int i0, i1, i2;
            if (!(s >> i0 >> i1 >> i2)) return "invalid OBJ triangle";
            tris.push_back(i0 - 1);
            tris.push_back(i1 - 1);
            tris.push_back(i2 - 1);
        }
    }

    // exact weld
    std::unordered_map<std::array<uint32_t, 3>, int, KeyHash> ids;
    std::vector<int> remap(raw.size());
    std::vector<V3> verts;
    for (size_t i = 0; i < raw.size(); i++) {
        const std::array<uint32_t, 3> k{ keyBits(raw[i].x), keyBits(raw[i].y), keyBits(raw[i].z) };
        auto it = ids.find(k);
        if (it == ids.end()) {
            it = ids.emplace(k, (int)verts.size()).first;
            verts.push_back(raw[i]);
        }
        remap[i] = it->second;
    }
    for (int& v : tris) {
        if (v < 0 || v >= (int)raw.size()) return "OBJ triangle index is out of range";
        v = remap[v];
    }
    const int nTris = (int)tris.size() / 3;

    out.verts.resize(3 * verts.size());
    for (size_t i = 0; i < verts.size(); i++) {
        out.verts[3 * i] = verts[i].x;
        out.verts[3 * i + 1] = verts[i].y;
        out.verts[3 * i + 2] = verts[i].z;
    }
    out.tris = tris;
    out.normals.assign(3 * (size_t)nTris, 0.f);

    std::vector<V3> nrm(nTris), lo(nTris), hi(nTris);
    for (int t = 0; t < nTris; t++) {
        const V3 a = verts[tris[3 * t]], b = verts[tris[3 * t + 1]], c = verts[tris[3 * t + 2]];
        const V3 cr = cross(b - a, c - a);
        const float l2 = lensq(cr);
        if (l2 <= 1e-12f) return "degenerate triangle in arena mesh";
        nrm[t] = cr * (1.f / sqrtf(l2));
        lo[t] = vmin(vmin(a, b), c);
        hi[t] = vmax(vmax(a, b), c);
        out.normals[3 * t] = nrm[t].x;
        out.normals[3 * t + 1] = nrm[t].y;
        out.normals[3 * t + 2] = nrm[t].z;
    }

    // uniform grid, counting pass then fill pass (ascending triangle order per cell)
    std::vector<int> count(kCells, 0);
    std::vector<std::array<int, 6>> range(nTris);
    for (int t = 0; t < nTris; t++) {
        int a0, a1, a2, b0, b1, b2;
        cellOf(lo[t], a0, a1, a2);
        cellOf(hi[t], b0, b1, b2);
        a0 = a0 - 1 < 0 ? 0 : a0 - 1;
        a1 = a1 - 1 < 0 ? 0 : a1 - 1;
        a2 = a2 - 1 < 0 ? 0 : a2 - 1;
        range[t] = { a0, a1, a2, b0, b1, b2 };
        for (int x = a0; x <= b0; x++)
            for (int y = a1; y <= b1; y++)
                for (int z = a2; z <= b2; z++) count[flatCell(x, y, z)]++;
    }
    out.cellStart.assign(kCells + 1, 0);
    for (int c = 0; c < kCells; c++) out.cellStart[c + 1] = out.cellStart[c] + count[c];
    out.cellTris.assign(out.cellStart[kCells], 0);
    std::fill(count.begin(), count.end(), 0);
    for (int t = 0; t < nTris; t++) {
        const auto& r = range[t];
        for (int x = r[0]; x <= r[3]; x++)
            for (int y = r[1]; y <= r[4]; y++)
                for (int z = r[2]; z <= r[5]; z++) {
                    const int c = flatCell(x, y, z);
                    out.cellTris[out.cellStart[c] + count[c]++] = t;
                }
    }

    // signed edge angles
    out.angles.assign(3 * (size_t)nTris, kBoundaryEdge);
    struct EdgeRec { int tri, slot, start, end; bool paired; };
    std::unordered_map<uint64_t, EdgeRec> edges;
    edges.reserve(3 * (size_t)nTris);
    for (int t = 0; t < nTris; t++) {
        for (int s = 0; s < 3; s++) {
            const int st = tris[3 * t + s], en = tris[3 * t + (s + 1) % 3];
            const uint64_t key = ((uint64_t)(uint32_t)std::min(st, en) << 32) | (uint32_t)std::max(st, en);
            auto it = edges.find(key);
            if (it == edges.end()) {
                edges.emplace(key, EdgeRec{ t, s, st, en, false });
                continue;
            }
            EdgeRec& first = it->second;
            if (first.paired) return "non-manifold edge in arena mesh";
            first.paired = true;
            if (first.start != en || first.end != st) return "inconsistent triangle winding in arena mesh";
            const V3 ev = verts[first.end] - verts[first.start];
            const float el = lensq(ev);
            if (el <= 1e-12f) return "degenerate edge in arena mesh";
            const V3 edge = ev * (1.f / sqrtf(el));
            const V3 na = nrm[first.tri], nb = nrm[t];
            const V3 nc = cross(na, nb);
            float nd = dot(na, nb);
            nd = nd < -1.f ? -1.f : (nd > 1.f ? 1.f : nd);
            float angle = 0.f;
            if (lensq(nc) <= 1e-4f) {
                if (nd < 0.f) return "opposing triangle normals in arena mesh";
            } else {
                angle = atan2f(dot(edge, nc), nd);
            }
            out.angles[3 * first.tri + first.slot] = angle;
            out.angles[3 * t + s] = angle;
        }
    }

    // device records, per triangle and per cell reference
    if (nTris >= kMaxArenaTris) return "arena mesh has more than 2^23 triangles";
    out.triRecords.assign(16 * (size_t)nTris, 0.f);
    const int nRefs = out.cellStart[kCells];
    out.records.assign(16 * (size_t)nRefs, 0.f);
    for (int t = 0; t < nTris; t++) {
        const V3 a = verts[tris[3 * t]], b = verts[tris[3 * t + 1]], c = verts[tris[3 * t + 2]];
        const V3 e1 = b - a, e2 = c - a;
        const bool horizontal = a.z == b.z && a.z == c.z && (a.z == 0.f || a.z == 2048.f);
        const bool sideWall = a.x == b.x && a.x == c.x && fabsf(a.x) == 4096.f;
        const uint32_t bits = (uint32_t)t | ((horizontal || sideWall) ? kPlaneFlag : 0u);
        float tag;
        std::memcpy(&tag, &bits, 4);
        const float rec[16] = { a.x, a.y, a.z, e1.x, e1.y, e1.z, e2.x, e2.y,
                                e2.z, b.x, b.y, b.z, c.x, c.y, c.z, tag };
        std::memcpy(&out.triRecords[16 * (size_t)t], rec, sizeof rec);
    }
    // Screening data of the contact search, per triangle (16 floats):
    //   box min xyz, n.x | box max xyz, n.y | n.z, n.v0, rayCond, rayTol |
    //   satS1, satS2, satS3, eps * longest edge
    // n is the unit normal of the plane through v0 along e1, e2 (the edges the
    // ray test uses).  The bounds come from the rounding analysis of the float
    // tests the screen stands in for (float32, no contraction, eps = 2^-24,
    // g = 16 eps, ray starts within T = 32768 of v0, rays at most 64 long,
    // s = |e1 x e2| / (|e1| |e2|)); each is enlarged by a quarter:
    //   rayTol   an accepted ray hit lies within (g (64 + T) + 2^-16) / s of
    //            the plane;
    //   rayCond  it lies within rayCond / |n.dir| of a point of the triangle,
    //            rayCond = g (3 T + |e1| + |e2| + 64) / s;
    //   satS*    the SAT normal axis, computed from vertices rotated with
    //            error at most 96 eps D (D the distance to the box centre),
    //            deviates from n by at most
    //            dn = d S1 + d^2 S2 + S3, d = 192 eps D + eps * longest edge,
    //            with a = |v1 - v0|, b = |v2 - v1|, 2A = |(v1 - v0) x (v2 - v1)|:
    //            S1 = 2 (a + b) / 2A, S2 = 2 / 2A, S3 = 12 eps a b / 2A + 4 eps.
    // A mesh with vertices beyond 8192 (the ray bound T no longer holds) gets
    // bounds that screen nothing.
    float vmaxAbs = 0.f;
    for (const V3& v : verts) vmaxAbs = std::max(vmaxAbs, std::max(std::fabs(v.x), std::max(std::fabs(v.y), std::fabs(v.z))));
    std::vector<float>& screen = out.triBoxes;
    screen.assign(16 * (size_t)nTris, 0.f);
    const double eps = std::ldexp(1.0, -24), g = 16.0 * eps, T = 32768.0, L = 64.0, grow = 1.25;
    for (int t = 0; t < nTris; t++) {
        const float* rec = &out.triRecords[16 * (size_t)t];
        const double ax = rec[0], ay = rec[1], az = rec[2];
        const double e1x = rec[3], e1y = rec[4], e1z = rec[5], e2x = rec[6], e2y = rec[7], e2z = rec[8];
        const double nx = e1y * e2z - e1z * e2y, ny = e1z * e2x - e1x * e2z, nz = e1x * e2y - e1y * e2x;
        const double nl = std::sqrt(nx * nx + ny * ny + nz * nz);
        const double l1 = std::sqrt(e1x * e1x + e1y * e1y + e1z * e1z);
        const double l2 = std::sqrt(e2x * e2x + e2y * e2y + e2z * e2z);
        const double sinA = nl / (l1 * l2);
        double rayTol = (g * (L + T) + std::ldexp(1.0, -16)) / sinA * grow + 0.05;
        double rayCond = g * (3.0 * T + l1 + l2 + L) / sinA * grow + 1e-3;
        // SAT edges from the vertices themselves
        const double p0x = rec[0], p0y = rec[1], p0z = rec[2], p1x = rec[9], p1y = rec[10], p1z = rec[11];
        const double p2x = rec[12], p2y = rec[13], p2z = rec[14];
        const double fx = p1x - p0x, fy = p1y - p0y, fz = p1z - p0z, hx = p2x - p1x, hy = p2y - p1y, hz = p2z - p1z;
        const double kx = p0x - p2x, ky = p0y - p2y, kz = p0z - p2z;
        const double sa = std::sqrt(fx * fx + fy * fy + fz * fz), sb = std::sqrt(hx * hx + hy * hy + hz * hz);
        const double sc = std::sqrt(kx * kx + ky * ky + kz * kz);
        const double cx = fy * hz - fz * hy, cy = fz * hx - fx * hz, cz = fx * hy - fy * hx;
        const double a2 = std::sqrt(cx * cx + cy * cy + cz * cz);
        double s1 = 2.0 * (sa + sb) / a2 * grow, s2 = 2.0 / a2 * grow, s3 = (12.0 * eps * sa * sb / a2 + 4.0 * eps) * grow;
        const double epsEdge = eps * std::max(sa, std::max(sb, sc)) * grow;
        if (!(vmaxAbs < 8192.f) || !(sinA > 1e-9) || !(rayTol < 1e30) || !(rayCond < 1e30)) rayTol = rayCond = 3e38;
        if (!(vmaxAbs < 8192.f) || !(a2 > 1e-9) || !(s1 < 1e30) || !(s2 < 1e30)) s1 = s2 = s3 = 3e38;
        const float f[16] = { lo[t].x, lo[t].y, lo[t].z, (float)(nx / nl),
                              hi[t].x, hi[t].y, hi[t].z, (float)(ny / nl),
                              (float)(nz / nl), (float)((nx * ax + ny * ay + nz * az) / nl), (float)rayCond, (float)rayTol,
                              (float)s1, (float)s2, (float)s3, (float)epsEdge };
        std::memcpy(&screen[16 * (size_t)t], f, sizeof f);
    }
    // ball candidate grid, also the cars' contact-search lists.  A ball only
    // tests triangles registered in the broadphase cells its box overlaps, a
    // car those of its own broadphase cell; each reference carries the
    // triangle's edge angles and its registration range (x0 x1 y0 y1 6 bits
    // each, z0 z1 4 bits) so that either can apply its rule itself, and the
    // triangle's contact-search screening data.
    {
        const double reach = (double)kBallRadius + (double)kBallArenaBreak + 1.0;
        auto fineRange = [&](int t, int (&a)[3], int (&b)[3]) {
            const double l[3] = { lo[t].x, lo[t].y, lo[t].z }, h[3] = { hi[t].x, hi[t].y, hi[t].z };
            const double o[3] = { kArenaMin.x, kArenaMin.y, kArenaMin.z };
            const int n[3] = { kFineX, kFineY, kFineZ };
            for (int k = 0; k < 3; k++) {
                a[k] = std::max(0, (int)std::floor((l[k] - reach - o[k]) / kFineCell));
                b[k] = std::min(n[k] - 1, (int)std::floor((h[k] + reach - o[k]) / kFineCell));
            }
        };
        std::vector<int> fcount(kFineCells + 1, 0);
        for (int t = 0; t < nTris; t++) {
            int a[3], b[3];
            fineRange(t, a, b);
            for (int z = a[2]; z <= b[2]; z++)
                for (int y = a[1]; y <= b[1]; y++)
                    for (int x = a[0]; x <= b[0]; x++) fcount[x + kFineX * (y + kFineY * z)]++;
        }
        out.fineStart.assign(kFineCells + 1, 0);
        for (int c = 0; c < kFineCells; c++) out.fineStart[c + 1] = out.fineStart[c] + fcount[c];
        const size_t nFine = (size_t)out.fineStart[kFineCells];
        out.fineRecords.assign(16 * nFine, 0.f);
        out.fineAux.assign(4 * nFine, 0.f);
        out.triAux.assign(4 * (size_t)nTris, 0.f);
        std::fill(fcount.begin(), fcount.end(), 0);
        for (int t = 0; t < nTris; t++) {
            int a[3], b[3];
            fineRange(t, a, b);
            const auto& r = range[t];
            const uint32_t reg = (uint32_t)r[0] | (uint32_t)r[3] << 6 | (uint32_t)r[1] << 12 | (uint32_t)r[4] << 18 |
                                 (uint32_t)r[2] << 24 | (uint32_t)r[5] << 28;
            std::memcpy(&out.triAux[4 * (size_t)t], &out.angles[3 * (size_t)t], 3 * sizeof(float));
            std::memcpy(&out.triAux[4 * (size_t)t + 3], &reg, sizeof reg);
            for (int z = a[2]; z <= b[2]; z++)
                for (int y = a[1]; y <= b[1]; y++)
                    for (int x = a[0]; x <= b[0]; x++) {
                        const int c = x + kFineX * (y + kFineY * z);
                        const size_t f = (size_t)out.fineStart[c] + fcount[c]++;
                        std::memcpy(&out.fineRecords[16 * f], &out.triRecords[16 * (size_t)t], 16 * sizeof(float));
                        std::memcpy(&out.fineAux[4 * f], &out.triAux[4 * (size_t)t], 4 * sizeof(float));
                    }
        }
    }
    // car candidate grid: the same rule with the car's reach, triangle
    // indices only, ascending within a cell
    {
        const double reach = (double)kCarGridReach;
        auto carRange = [&](int t, int (&a)[3], int (&b)[3]) {
            const double l[3] = { lo[t].x, lo[t].y, lo[t].z }, h[3] = { hi[t].x, hi[t].y, hi[t].z };
            const double o[3] = { kArenaMin.x, kArenaMin.y, kArenaMin.z };
            const int n[3] = { kCarX, kCarY, kCarZ };
            for (int k = 0; k < 3; k++) {
                a[k] = std::max(0, (int)std::floor((l[k] - reach - o[k]) / kCarCell));
                b[k] = std::min(n[k] - 1, (int)std::floor((h[k] + reach - o[k]) / kCarCell));
            }
        };
        std::vector<int> ccount(kCarCells + 1, 0);
        for (int t = 0; t < nTris; t++) {
            int a[3], b[3];
            carRange(t, a, b);
            for (int z = a[2]; z <= b[2]; z++)
                for (int y = a[1]; y <= b[1]; y++)
                    for (int x = a[0]; x <= b[0]; x++) ccount[x + kCarX * (y + kCarY * z)]++;
        }
        out.carStart.assign(kCarCells + 1, 0);
        for (int c = 0; c < kCarCells; c++) out.carStart[c + 1] = out.carStart[c] + ccount[c];
        out.carTris.assign((size_t)out.carStart[kCarCells], 0);
        std::fill(ccount.begin(), ccount.end(), 0);
        for (int t = 0; t < nTris; t++) {
            int a[3], b[3];
            carRange(t, a, b);
            for (int z = a[2]; z <= b[2]; z++)
                for (int y = a[1]; y <= b[1]; y++)
                    for (int x = a[0]; x <= b[0]; x++) {
                        const int c = x + kCarX * (y + kCarY * z);
                        out.carTris[(size_t)out.carStart[c] + ccount[c]++] = t;
                    }
        }
    }
    for (int r = 0; r < nRefs; r++)
        std::memcpy(&out.records[16 * (size_t)r], &out.triRecords[16 * (size_t)out.cellTris[r]], 16 * sizeof(float));
    return "";
}

// The reference reads the count, then per triangle mesh, order, three edge
// angles, flags and three native vertices, all whitespace separated with
// stream extraction, and checks the stream only once, after the last
// triangle (src/ArenaMesh.cu:69-99).  A file that cannot be opened reads as a
// count of 0, so it fails the count check too.
std::string readArenaMetadata(const char* path, HostArena& out)
{
    const int nTris = (int)(out.tris.size() / 3);
    std::ifstream file(path);
    int count = 0;
    file >> count;
    if (count != nTris) return "CARL arena metadata triangle count mismatch";
    out.nativeRecords.assign(16 * (size_t)nTris, 0.f);
    for (int t = 0; t < nTris; t++) {
        int mesh = 0, order = 0, flags = 0;
        float a[3] = {}, v[9] = {};
        file >> mesh >> order >> a[0] >> a[1] >> a[2] >> flags;
        for (float& x : v) file >> x;
        // the reference's order key, mesh * 10000 + order, in 32-bit
        // arithmetic
        const int32_t key = (int32_t)((uint32_t)mesh * 10000u + (uint32_t)order);
        float* r = &out.nativeRecords[16 * (size_t)t];
        const int32_t ints[3] = { key, mesh, flags };
        for (int k = 0; k < 3; k++) {
            r[4 * k] = v[3 * k];
            r[4 * k + 1] = v[3 * k + 1];
            r[4 * k + 2] = v[3 * k + 2];
            std::memcpy(&r[4 * k + 3], &ints[k], sizeof(int32_t));
        }
        r[12] = a[0];
        r[13] = a[1];
        r[14] = a[2];
    }
    if (!file) return "Invalid CARL arena metadata";
    return "";
}

}  // namespace carl
