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
    std::vector<float> refBoxes;    // 16 floats per cell reference: contact-search screening data
    std::vector<float> refAngles;   // 4 per cell reference: the triangle's signed edge angles xyz, 0
    std::vector<int> fineStart;     // kFineCells + 1 offsets into fineRecords (in references)
    std::vector<float> fineRecords; // 16 floats per ball-grid reference (record layout), ascending per cell
    std::vector<float> fineAux;     // 4 per ball-grid reference: edge angles xyz, registration range (bits)
};

// Parse, weld and index the mesh.  Returns "" on success, else the error text.
std::string buildArena(const std::string& objPath, HostArena& out);

// Locate arena.obj: $CARL_ARENA_OBJ, then assets/arena.obj next to the package.
std::string findArenaObj(const std::string& libraryDir);

}  // namespace carl
