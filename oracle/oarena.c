/*
 * oarena.c - arena mesh construction for the CPU oracle.
 *
 * TEST INFRASTRUCTURE (see omath.h).  Restates the host mesh build of the
 * reference:
 *   OBJ parse with the x/y swap        include/Arena/ObjLoader.cuh:91-126
 *   exact-bit vertex weld (-0 == +0)   include/Arena/ObjLoader.cuh:49-89
 *   face normals, bounds               include/Arena/TriMesh.cuh:26-69
 *   48x48x10 grid, cells [cell(min)-1, cell(max)]
 *                                      include/Arena/BroadPhaseGrid.cuh:11-78
 *   signed edge angles                 include/Arena/EdgeInfo.cuh:60-125
 *   native mesh metadata               src/ArenaMesh.cu:69-124
 */
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include "ointernal.h"

static void set_err(char* err, int len, const char* msg)
{
    if (err && len > 0) { strncpy(err, msg, (size_t)len - 1); err[len - 1] = 0; }
}

void oarena_cell3(V3 p, int* cx, int* cy, int* cz)
{
    /* ((p - ARENA_MIN) / CELL_SIZE).max(0).min(GRID_DIMS - 1).toInt3() */
    float x = (p.x - K_ARENA_MIN.x) / K_CELL_X;
    float y = (p.y - K_ARENA_MIN.y) / K_CELL_Y;
    float z = (p.z - K_ARENA_MIN.z) / K_CELL_Z;
    x = o_min(o_max(x, 0.f), K_GRID_DIMS.x - 1.f);
    y = o_min(o_max(y, 0.f), K_GRID_DIMS.y - 1.f);
    z = o_min(o_max(z, 0.f), K_GRID_DIMS.z - 1.f);
    *cx = (int)x; *cy = (int)y; *cz = (int)z;
}

int oarena_flat(int cx, int cy, int cz) { return cx + cy * GRID_X + cz * GRID_X * GRID_Y; }

static uint32_t fbits(float v)
{
    if (v == 0.f) v = 0.f;
    uint32_t u;
    memcpy(&u, &v, 4);
    return u;
}

typedef struct { uint32_t k[3]; int idx; } WeldKey;

static int weld_cmp(const void* a, const void* b)
{
    const WeldKey* x = (const WeldKey*)a;
    const WeldKey* y = (const WeldKey*)b;
    for (int i = 0; i < 3; i++) {
        if (x->k[i] != y->k[i]) return x->k[i] < y->k[i] ? -1 : 1;
    }
    return x->idx < y->idx ? -1 : (x->idx > y->idx);
}

/* edge table: open addressing on (lo, hi) vertex pairs */
typedef struct { int lo, hi, tri, slot, start, end, paired, used; } EdgeSlot;

static uint32_t edge_hash(int lo, int hi)
{
    return o_hash32((uint32_t)lo * 2654435761u ^ (uint32_t)hi);
}

void oarena_free(OArena* a)
{
    if (!a) return;
    free(a->verts); free(a->tris); free(a->norms); free(a->aabbMin);
    free(a->aabbMax); free(a->angs); free(a->cellTris);
    free(a->nkey); free(a->nmesh); free(a->nflags); free(a->nverts); free(a->nangs); free(a->ballTris);
    free(a);
}

OArena* oarena_load(const char* path, char* err, int errLen)
{
    FILE* f = fopen(path, "r");
    if (!f) { set_err(err, errLen, "failed to open assets/arena.obj"); return NULL; }

    int capV = 8192, capT = 16384, nV = 0, nT = 0;
    V3* verts = (V3*)malloc(sizeof(V3) * (size_t)capV);
    int* tris = (int*)malloc(sizeof(int) * 3 * (size_t)capT);
    char line[512];
    while (fgets(line, sizeof line, f)) {
        char type[16];
        int off = 0;
        if (sscanf(line, "%15s%n", type, &off) != 1) continue;
        if (strcmp(type, "v") == 0) {
            float x, y, z;
            /* the source OBJ swaps the horizontal axes */
            if (sscanf(line + off, "%f %f %f", &y, &x, &z) != 3) {
                set_err(err, errLen, "invalid OBJ vertex");
                fclose(f); free(verts); free(tris); return NULL;
            }
            if (nV == capV) { capV *= 2; verts = (V3*)realloc(verts, sizeof(V3) * (size_t)capV); }
            verts[nV++] = v3(x, y, z);
        } else if (strcmp(type, "f") == 0) {
            int a, b, c;
            if (sscanf(line + off, "%d %d %d", &a, &b, &c) != 3) {
                set_err(err, errLen, "invalid OBJ triangle");
                fclose(f); free(verts); free(tris); return NULL;
            }
            if (nT == capT) { capT *= 2; tris = (int*)realloc(tris, sizeof(int) * 3 * (size_t)capT); }
            tris[3 * nT] = a - 1; tris[3 * nT + 1] = b - 1; tris[3 * nT + 2] = c - 1;
            nT++;
        }
    }
    fclose(f);

    /* weld: welded vertices keep the order of first occurrence */
    WeldKey* keys = (WeldKey*)malloc(sizeof(WeldKey) * (size_t)(nV ? nV : 1));
    for (int i = 0; i < nV; i++) {
        keys[i].k[0] = fbits(verts[i].x); keys[i].k[1] = fbits(verts[i].y); keys[i].k[2] = fbits(verts[i].z);
        keys[i].idx = i;
    }
    qsort(keys, (size_t)nV, sizeof(WeldKey), weld_cmp);
    int* rep = (int*)malloc(sizeof(int) * (size_t)(nV ? nV : 1));
    for (int i = 0; i < nV;) {
        int j = i;
        while (j < nV && memcmp(keys[j].k, keys[i].k, sizeof keys[i].k) == 0) j++;
        for (int m = i; m < j; m++) rep[keys[m].idx] = keys[i].idx; /* smallest index of the group */
        i = j;
    }
    int* newId = (int*)malloc(sizeof(int) * (size_t)(nV ? nV : 1));
    int nW = 0;
    V3* welded = (V3*)malloc(sizeof(V3) * (size_t)(nV ? nV : 1));
    for (int i = 0; i < nV; i++) {
        if (rep[i] == i) { newId[i] = nW; welded[nW++] = verts[i]; }
    }
    for (int t = 0; t < 3 * nT; t++) {
        const int v = tris[t];
        if (v < 0 || v >= nV) {
            set_err(err, errLen, "OBJ triangle index is out of range");
            free(keys); free(rep); free(newId); free(welded); free(verts); free(tris);
            return NULL;
        }
        tris[t] = newId[rep[v]];
    }
    free(keys); free(rep); free(newId); free(verts);

    OArena* a = (OArena*)calloc(1, sizeof(OArena));
    a->nVerts = nW; a->nTris = nT; a->verts = welded; a->tris = tris;
    a->norms = (V3*)malloc(sizeof(V3) * (size_t)nT);
    a->aabbMin = (V3*)malloc(sizeof(V3) * (size_t)nT);
    a->aabbMax = (V3*)malloc(sizeof(V3) * (size_t)nT);
    a->angs = (V3*)malloc(sizeof(V3) * (size_t)nT);

    for (int t = 0; t < nT; t++) {
        const V3 p0 = welded[tris[3 * t]], p1 = welded[tris[3 * t + 1]], p2 = welded[tris[3 * t + 2]];
        const V3 cr = vcross(vsub(p1, p0), vsub(p2, p0));
        const float l = vlensq(cr);
        if (l <= 1e-12f) {
            set_err(err, errLen, "degenerate triangle in arena mesh");
            oarena_free(a); return NULL;
        }
        a->norms[t] = vscale(cr, 1.f / sqrtf(l));
        a->aabbMin[t] = vmin(vmin(p0, p1), p2);
        a->aabbMax[t] = vmax(vmax(p0, p1), p2);
    }

    /* grid: two passes so that each cell lists its triangles in ascending order */
    int* counts = (int*)calloc(N_CELLS, sizeof(int));
    int (*lo)[3] = malloc(sizeof(int[3]) * (size_t)nT);
    int (*hi)[3] = malloc(sizeof(int[3]) * (size_t)nT);
    for (int t = 0; t < nT; t++) {
        oarena_cell3(a->aabbMin[t], &lo[t][0], &lo[t][1], &lo[t][2]);
        for (int k = 0; k < 3; k++) { lo[t][k] -= 1; if (lo[t][k] < 0) lo[t][k] = 0; }
        oarena_cell3(a->aabbMax[t], &hi[t][0], &hi[t][1], &hi[t][2]);
        for (int x = lo[t][0]; x <= hi[t][0]; x++)
            for (int y = lo[t][1]; y <= hi[t][1]; y++)
                for (int z = lo[t][2]; z <= hi[t][2]; z++) counts[oarena_flat(x, y, z)]++;
    }
    a->cellPrefix[0] = 0;
    for (int c = 0; c < N_CELLS; c++) a->cellPrefix[c + 1] = a->cellPrefix[c] + counts[c];
    a->cellTris = (int*)malloc(sizeof(int) * (size_t)(a->cellPrefix[N_CELLS] ? a->cellPrefix[N_CELLS] : 1));
    memset(counts, 0, sizeof(int) * N_CELLS);
    for (int t = 0; t < nT; t++) {
        for (int x = lo[t][0]; x <= hi[t][0]; x++)
            for (int y = lo[t][1]; y <= hi[t][1]; y++)
                for (int z = lo[t][2]; z <= hi[t][2]; z++) {
                    const int c = oarena_flat(x, y, z);
                    a->cellTris[a->cellPrefix[c] + counts[c]++] = t;
                }
    }
    free(counts); free(lo); free(hi);

    /* signed edge angles */
    for (int t = 0; t < nT; t++) a->angs[t] = v3(K_BOUNDARY_EDGE_ANGLE, K_BOUNDARY_EDGE_ANGLE, K_BOUNDARY_EDGE_ANGLE);
    const int cap = 1 << 17;
    EdgeSlot* table = (EdgeSlot*)calloc((size_t)cap, sizeof(EdgeSlot));
    const char* fail = NULL;
    for (int t = 0; t < nT && !fail; t++) {
        for (int s = 0; s < 3 && !fail; s++) {
            const int st = tris[3 * t + s], en = tris[3 * t + (s + 1) % 3];
            const int elo = st < en ? st : en, ehi = st < en ? en : st;
            uint32_t h = edge_hash(elo, ehi) & (uint32_t)(cap - 1);
            while (table[h].used && !(table[h].lo == elo && table[h].hi == ehi)) h = (h + 1) & (uint32_t)(cap - 1);
            EdgeSlot* e = &table[h];
            if (!e->used) {
                e->used = 1; e->lo = elo; e->hi = ehi; e->tri = t; e->slot = s; e->start = st; e->end = en;
                continue;
            }
            if (e->paired) { fail = "non-manifold edge in arena mesh"; break; }
            e->paired = 1;
            if (e->start != en || e->end != st) { fail = "inconsistent triangle winding in arena mesh"; break; }
            /* signedEdgeAngle(verts[first.start], verts[first.end], n[first], n[this]) */
            const V3 ev = vsub(welded[e->end], welded[e->start]);
            const float el = vlensq(ev);
            if (el <= 1e-12f) { fail = "degenerate edge in arena mesh"; break; }
            const V3 edge = vscale(ev, 1.f / sqrtf(el));
            const V3 nA = a->norms[e->tri], nB = a->norms[t];
            const V3 nc = vcross(nA, nB);
            float nd = vdot(nA, nB);
            nd = nd < -1.f ? -1.f : (nd > 1.f ? 1.f : nd);
            float angle;
            if (vlensq(nc) <= 1e-4f) {
                if (nd < 0.f) { fail = "opposing triangle normals in arena mesh"; break; }
                angle = 0.f;
            } else {
                angle = atan2f(vdot(edge, nc), nd);
            }
            vset(&a->angs[e->tri], e->slot, angle);
            vset(&a->angs[t], s, angle);
        }
    }
    free(table);
    if (fail) { set_err(err, errLen, fail); oarena_free(a); return NULL; }
    return a;
}

/* src/ArenaMesh.cu:69-99: the count, then per triangle mesh, order, three
 * edge angles, flags and three vertices, read one after another; the read
 * state is checked after the last triangle only.  A file that does not open
 * reads as count 0.  Then (:109-124) each cell's ball list is sorted by the
 * order key; triangles of equal keys, whose order the reference leaves to
 * std::sort, go by triangle index here. */
typedef struct { int key, tri; } BallKey;

static int ball_key_cmp(const void* x, const void* y)
{
    const BallKey* a = (const BallKey*)x;
    const BallKey* b = (const BallKey*)y;
    if (a->key != b->key) return a->key < b->key ? -1 : 1;
    return a->tri < b->tri ? -1 : (a->tri > b->tri);
}

int oarena_load_metadata(OArena* a, const char* path, char* err, int errLen)
{
    FILE* f = fopen(path, "r");
    int count = 0;
    if (!f || fscanf(f, "%d", &count) != 1) count = 0;
    if (count != a->nTris) {
        if (f) fclose(f);
        set_err(err, errLen, "CARL arena metadata triangle count mismatch");
        return 0;
    }
    const int n = a->nTris;
    a->nkey = (int*)calloc((size_t)n, sizeof(int));
    a->nmesh = (int*)calloc((size_t)n, sizeof(int));
    a->nflags = (int*)calloc((size_t)n, sizeof(int));
    a->nverts = (V3*)calloc(3 * (size_t)n, sizeof(V3));
    a->nangs = (V3*)calloc((size_t)n, sizeof(V3));
    int ok = 1;
    for (int t = 0; t < n && ok; t++) {
        int mesh, order, flags;
        float ax, ay, az, v[9];
        ok = fscanf(f, "%d %d %f %f %f %d", &mesh, &order, &ax, &ay, &az, &flags) == 6;
        for (int k = 0; k < 9 && ok; k++) ok = fscanf(f, "%f", &v[k]) == 1;
        if (!ok) break;
        /* mesh * 10000 + order in 32-bit arithmetic */
        a->nkey[t] = (int)((uint32_t)mesh * 10000u + (uint32_t)order);
        a->nmesh[t] = mesh;
        a->nflags[t] = flags;
        a->nangs[t] = v3(ax, ay, az);
        for (int k = 0; k < 3; k++) a->nverts[3 * t + k] = v3(v[3 * k], v[3 * k + 1], v[3 * k + 2]);
    }
    fclose(f);
    if (!ok) {
        set_err(err, errLen, "Invalid CARL arena metadata");
        return 0;
    }
    const int refs = a->cellPrefix[N_CELLS];
    a->ballTris = (int*)malloc(sizeof(int) * (size_t)(refs ? refs : 1));
    BallKey* keys = (BallKey*)malloc(sizeof(BallKey) * (size_t)(refs ? refs : 1));
    for (int r = 0; r < refs; r++) { keys[r].tri = a->cellTris[r]; keys[r].key = a->nkey[a->cellTris[r]]; }
    for (int c = 0; c < N_CELLS; c++) {
        const int lo = a->cellPrefix[c], cnt = a->cellPrefix[c + 1] - lo;
        if (cnt > 1) qsort(keys + lo, (size_t)cnt, sizeof(BallKey), ball_key_cmp);
    }
    for (int r = 0; r < refs; r++) a->ballTris[r] = keys[r].tri;
    free(keys);
    a->native = 1;
    return 1;
}
