// ============================================================================
//  formats.hpp — host-side writer of the MARS v1 graph file, shared by the
//  array entry points (formats.cpp) and the device-graph checkpoint (api.hip).
//
//  MARS v1 (the layout of the reference's persistence.h:8-18): "MARS", uint32
//  version 1, int32 num_nodes, num_edges, embedding_dim, then row_offsets
//  (num_nodes + 1 int32), col_indices (num_edges int32), embeddings
//  (num_nodes x dim float), modalities (num_nodes int32), timestamps
//  (num_nodes float), and the FNV-1a 64-bit hash of every preceding byte.
//  Native (little-endian) byte order, as the reference writes it.
// ============================================================================
#pragma once

#include <cstddef>
#include <cstdint>
#include <cstdio>
#include <string>

namespace mars {

constexpr uint32_t kGraphFileVersion = 1;
constexpr size_t kGraphFileHeader = 20;        // magic, version, three sizes

// FNV-1a, 64 bit (offset basis and prime of the published FNV-1a definition).
constexpr uint64_t kFnvOffset = 0xCBF29CE484222325ull;
constexpr uint64_t kFnvPrime = 0x00000100000001B3ull;
uint64_t fnv1a_update(uint64_t h, const void* data, size_t len);

// Expected byte size of a MARS v1 file with these sizes (checksum included).
uint64_t graph_file_bytes(int32_t num_nodes, int32_t num_edges, int32_t dim);

// Writes a MARS v1 file piece by piece, hashing as it goes. Every call returns
// MARS_OK or an error code (with the thread's error message set).
class GraphFileWriter {
public:
    GraphFileWriter() = default;
    GraphFileWriter(const GraphFileWriter&) = delete;
    GraphFileWriter& operator=(const GraphFileWriter&) = delete;
    ~GraphFileWriter();
    int open(const char* path, int32_t num_nodes, int32_t num_edges, int32_t dim);
    int put(const void* data, size_t bytes);   // the next bytes of the arrays, in file order
    int finish();                              // checks the byte count, appends the hash, closes

private:
    FILE* f_ = nullptr;
    uint64_t hash_ = kFnvOffset;
    uint64_t written_ = 0;
    uint64_t expected_ = 0;
    std::string path_;
};

}  // namespace mars
