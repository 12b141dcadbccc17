// arena.h - host-side construction of the soccar collision mesh.
#pragma once

#include <cstdint>
#include <string>
#include <vector>

namespace carl {

struct HostArena {
    std::vector<float> verts;       // 3 per welded vertex
    std::vector<int> tris;          // 3 per triangle
    std::vector<float> normals;     // 3 per triangle
    std::vector<float> angles;      // 3 per triangle (signed edge angles)
    std::vector<int> cellStart;     // kCells + 1
    std::vector<int> cellTris;      // triangle per cell reference, ascending within a cell
    std::vector<float> records;     // 16 floats per cell reference (device layout, see state.h)
    std::vector<float> triRecords;  // the same 16 floats per triangle, by triangle index
    std::vector<float> triBoxes;    // 16 floats per triangle: contact-search screening data
    std::vector<float> triAux;      // 4 per triangle: edge angles xyz, registration range (bits)
    std::vector<int> fineStart;     // kFineCells + 1 offsets into fineRecords (in references)
    std::vector<float> fineRecords; // 16 floats per ball-grid reference (record layout), ascending per cell
    std::vector<float> fineAux;     // 4 per ball-grid reference: edge angles xyz, registration range (bits)
    std::vector<int> carStart;      // kCarCells + 1 offsets into carTris
    std::vector<int> carTris;       // triangle per car-grid reference, ascending within a cell
    // native mesh metadata (only with CARL_ARENA_METADATA), 16 floats per
    // triangle: native vertex 0 xyz, order key (int bits, mesh * 10000 +
    // order); vertex 1 xyz, native mesh (int bits); vertex 2 xyz, edge flags
    // (int bits); native edge angles xyz, 0.  Vertices in Bullet units.
    std::vector<float> nativeRecords;
};

// Parse, weld and index the mesh.  Returns "" on success, else the error text.
std::string buildArena(const std::string& objPath, HostArena& out);

// Read the native mesh metadata file (the format tools/arena_metadata.py
// writes) into out.nativeRecords.  Returns "" on success, else the reference's
// error text.
std::string readArenaMetadata(const char* path, HostArena& out);

// Locate arena.obj: $CARL_ARENA_OBJ, then assets/arena.obj next to the package.
std::string findArenaObj(const std::string& libraryDir);

}  // namespace carl
