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
    if (nTris > kMaxArenaTris) return "arena mesh has more than 65535 triangles";
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
    for (int r = 0; r < nRefs; r++)
        std::memcpy(&out.records[16 * (size_t)r], &out.triRecords[16 * (size_t)out.cellTris[r]], 16 * sizeof(float));
    return "";
}

}  // namespace carl
