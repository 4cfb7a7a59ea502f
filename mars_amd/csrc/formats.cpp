// ============================================================================
//  formats.cpp — files on either side of the path, host code:
//    * MARS v1 graph files (layout of the reference's persistence.h:8-18; save /
//      load semantics of src/persistence.cpp: a file is accepted only if its
//      FNV-1a hash, magic, version and exact size all check);
//    * the KIDS binary corpus (layout of demos/embodied_scene/bench_kids_sweep.cu:
//      29-37, writer :84-102, reader scripts/bench_kids_ball_cuvs_cagra.py:49-60).
//  The device-graph checkpoint (mars_graph_save) is in api.hip on the same writer.
// ============================================================================
#include "formats.hpp"

#include "mars_amd.h"

#include <cstring>
#include <vector>

namespace mars {

int set_error(int code, const char* fmt, ...);

namespace {

constexpr char kGraphMagic[4] = {'M', 'A', 'R', 'S'};
constexpr uint32_t kKidsMagic = 0x5344494Bu;   // bytes "KIDS" in little-endian order
constexpr uint32_t kKidsVersion = 1;
constexpr size_t kChunk = size_t(64) << 20;   // read / hash granularity

struct File {
    FILE* f = nullptr;
    ~File() {
        if (f) std::fclose(f);
    }
};

int64_t file_size(FILE* f) {
    if (fseeko(f, 0, SEEK_END) != 0) return -1;
    const int64_t n = int64_t(ftello(f));
    if (fseeko(f, 0, SEEK_SET) != 0) return -1;
    return n;
}

// Reads bytes into dst in chunks, hashing them into *h (when h != null).
int read_hashed(FILE* f, void* dst, uint64_t bytes, uint64_t* h, const char* path) {
    auto* p = static_cast<uint8_t*>(dst);
    while (bytes > 0) {
        const size_t n = size_t(bytes < kChunk ? bytes : kChunk);
        if (std::fread(p, 1, n, f) != n) return set_error(MARS_ERR_INVALID, "%s: short read", path);
        if (h) *h = fnv1a_update(*h, p, n);
        p += n;
        bytes -= n;
    }
    return MARS_OK;
}

int write_all(FILE* f, const void* data, uint64_t bytes, const char* path) {
    if (bytes > 0 && std::fwrite(data, 1, size_t(bytes), f) != size_t(bytes))
        return set_error(MARS_ERR_INVALID, "%s: write failed", path);
    return MARS_OK;
}

struct GraphHeader {
    int32_t n = 0, e = 0, d = 0;
};

// Reads and checks the 20-byte header and the file size.
int read_graph_header(FILE* f, const char* path, GraphHeader* hd, uint8_t raw[kGraphFileHeader]) {
    const int64_t size = file_size(f);
    if (size < int64_t(kGraphFileHeader + sizeof(uint64_t)))
        return set_error(MARS_ERR_INVALID, "%s: %lld bytes, too short for a MARS v1 file", path, (long long)size);
    if (std::fread(raw, 1, kGraphFileHeader, f) != kGraphFileHeader)
        return set_error(MARS_ERR_INVALID, "%s: short read", path);
    if (std::memcmp(raw, kGraphMagic, 4) != 0) return set_error(MARS_ERR_INVALID, "%s: not a MARS file", path);
    uint32_t version = 0;
    std::memcpy(&version, raw + 4, 4);
    if (version != kGraphFileVersion)
        return set_error(MARS_ERR_UNSUPPORTED, "%s: MARS file version %u (this build reads 1)", path, version);
    std::memcpy(&hd->n, raw + 8, 4);
    std::memcpy(&hd->e, raw + 12, 4);
    std::memcpy(&hd->d, raw + 16, 4);
    if (hd->n < 0 || hd->e < 0 || hd->d < 0)
        return set_error(MARS_ERR_INVALID, "%s: negative size in the header", path);
    if (uint64_t(size) != graph_file_bytes(hd->n, hd->e, hd->d))
        return set_error(MARS_ERR_INVALID, "%s: %lld bytes, the header describes %llu", path, (long long)size,
                         (unsigned long long)graph_file_bytes(hd->n, hd->e, hd->d));
    return MARS_OK;
}

uint64_t kids_file_bytes(int32_t n, int32_t d) {
    return 16 + uint64_t(n) * uint64_t(d) * 4 + uint64_t(n) * 12;
}

int read_kids_header(FILE* f, const char* path, int32_t* n, int32_t* d) {
    const int64_t size = file_size(f);
    uint8_t raw[16];
    if (size < 16 || std::fread(raw, 1, 16, f) != 16)
        return set_error(MARS_ERR_INVALID, "%s: too short for a KIDS corpus", path);
    uint32_t magic = 0;
    std::memcpy(&magic, raw, 4);
    if (magic != kKidsMagic) return set_error(MARS_ERR_INVALID, "%s: bad magic 0x%08x", path, magic);
    std::memcpy(n, raw + 8, 4);
    std::memcpy(d, raw + 12, 4);
    if (*n < 0 || *d < 0) return set_error(MARS_ERR_INVALID, "%s: negative size in the header", path);
    if (uint64_t(size) != kids_file_bytes(*n, *d))
        return set_error(MARS_ERR_INVALID, "%s: %lld bytes, the header describes %llu", path, (long long)size,
                         (unsigned long long)kids_file_bytes(*n, *d));
    return MARS_OK;
}

}  // namespace

uint64_t fnv1a_update(uint64_t h, const void* data, size_t len) {
    const auto* b = static_cast<const uint8_t*>(data);
    size_t i = 0;
    for (; i + 8 <= len; i += 8) {
        uint64_t w;
        std::memcpy(&w, b + i, 8);
        for (int k = 0; k < 8; ++k) h = (h ^ ((w >> (8 * k)) & 0xFFu)) * kFnvPrime;
    }
    for (; i < len; ++i) h = (h ^ b[i]) * kFnvPrime;
    return h;
}

uint64_t graph_file_bytes(int32_t num_nodes, int32_t num_edges, int32_t dim) {
    const uint64_t n = uint64_t(num_nodes), e = uint64_t(num_edges), d = uint64_t(dim);
    return kGraphFileHeader + (n + 1) * 4 + e * 4 + n * d * 4 + n * 4 + n * 4 + sizeof(uint64_t);
}

GraphFileWriter::~GraphFileWriter() {
    if (f_) std::fclose(f_);
}

int GraphFileWriter::open(const char* path, int32_t num_nodes, int32_t num_edges, int32_t dim) {
    if (!path) return set_error(MARS_ERR_INVALID, "null path");
    if (num_nodes < 0 || num_edges < 0 || dim < 0)
        return set_error(MARS_ERR_INVALID, "negative size (%d nodes, %d edges, dim %d)", num_nodes, num_edges, dim);
    path_ = path;
    f_ = std::fopen(path, "wb");
    if (!f_) return set_error(MARS_ERR_INVALID, "%s: cannot open for writing", path);
    expected_ = graph_file_bytes(num_nodes, num_edges, dim) - sizeof(uint64_t);
    hash_ = kFnvOffset;
    written_ = 0;
    uint8_t raw[kGraphFileHeader];
    std::memcpy(raw, kGraphMagic, 4);
    std::memcpy(raw + 4, &kGraphFileVersion, 4);
    std::memcpy(raw + 8, &num_nodes, 4);
    std::memcpy(raw + 12, &num_edges, 4);
    std::memcpy(raw + 16, &dim, 4);
    return put(raw, sizeof(raw));
}

int GraphFileWriter::put(const void* data, size_t bytes) {
    if (!f_) return set_error(MARS_ERR_INVALID, "graph file not open");
    if (written_ + bytes > expected_)
        return set_error(MARS_ERR_INVALID, "%s: more bytes than the header describes", path_.c_str());
    if (int rc = write_all(f_, data, bytes, path_.c_str())) return rc;
    hash_ = fnv1a_update(hash_, data, bytes);
    written_ += bytes;
    return MARS_OK;
}

int GraphFileWriter::finish() {
    if (!f_) return set_error(MARS_ERR_INVALID, "graph file not open");
    if (written_ != expected_)
        return set_error(MARS_ERR_INVALID, "%s: %llu bytes written, the header describes %llu", path_.c_str(),
                         (unsigned long long)written_, (unsigned long long)expected_);
    if (int rc = write_all(f_, &hash_, sizeof(hash_), path_.c_str())) return rc;
    const int closed = std::fclose(f_);
    f_ = nullptr;
    if (closed != 0) return set_error(MARS_ERR_INVALID, "%s: close failed", path_.c_str());
    return MARS_OK;
}

}  // namespace mars

using mars::set_error;

extern "C" {

int mars_fnv1a64(const void* data, int64_t len, uint64_t* out) {
    if (!out || len < 0 || (len > 0 && !data)) return set_error(MARS_ERR_INVALID, "bad arguments");
    *out = mars::fnv1a_update(mars::kFnvOffset, data, size_t(len));
    return MARS_OK;
}

int mars_graph_file_save(const char* path, int32_t num_nodes, int32_t num_edges, int32_t dim,
                         const int32_t* row_offsets, const int32_t* col_indices, const float* embeddings,
                         const int32_t* modalities, const float* timestamps) {
    if (!row_offsets || (num_edges > 0 && !col_indices) ||
        (num_nodes > 0 && (!modalities || !timestamps || (dim > 0 && !embeddings))))
        return set_error(MARS_ERR_INVALID, "null array");
    mars::GraphFileWriter w;
    const uint64_t n = uint64_t(num_nodes > 0 ? num_nodes : 0);
    int rc = w.open(path, num_nodes, num_edges, dim);
    if (!rc) rc = w.put(row_offsets, (n + 1) * 4);
    if (!rc) rc = w.put(col_indices, uint64_t(num_edges) * 4);
    if (!rc) rc = w.put(embeddings, n * uint64_t(dim) * 4);
    if (!rc) rc = w.put(modalities, n * 4);
    if (!rc) rc = w.put(timestamps, n * 4);
    if (!rc) rc = w.finish();
    return rc;
}

int mars_graph_file_info(const char* path, int32_t* num_nodes, int32_t* num_edges, int32_t* dim) {
    if (!path || !num_nodes || !num_edges || !dim) return set_error(MARS_ERR_INVALID, "null argument");
    mars::File f;
    f.f = std::fopen(path, "rb");
    if (!f.f) return set_error(MARS_ERR_INVALID, "%s: cannot open", path);
    mars::GraphHeader hd;
    uint8_t raw[mars::kGraphFileHeader];
    if (int rc = mars::read_graph_header(f.f, path, &hd, raw)) return rc;
    *num_nodes = hd.n;
    *num_edges = hd.e;
    *dim = hd.d;
    return MARS_OK;
}

int mars_graph_file_load(const char* path, int32_t num_nodes, int32_t num_edges, int32_t dim,
                         int32_t* row_offsets, int32_t* col_indices, float* embeddings, int32_t* modalities,
                         float* timestamps) {
    if (!path) return set_error(MARS_ERR_INVALID, "null path");
    mars::File f;
    f.f = std::fopen(path, "rb");
    if (!f.f) return set_error(MARS_ERR_INVALID, "%s: cannot open", path);
    mars::GraphHeader hd;
    uint8_t raw[mars::kGraphFileHeader];
    if (int rc = mars::read_graph_header(f.f, path, &hd, raw)) return rc;
    if (hd.n != num_nodes || hd.e != num_edges || hd.d != dim)
        return set_error(MARS_ERR_INVALID, "%s holds %d nodes, %d edges, dim %d (asked %d, %d, %d)", path, hd.n, hd.e,
                         hd.d, num_nodes, num_edges, dim);
    const uint64_t n = uint64_t(hd.n);
    if (!row_offsets || (hd.e > 0 && !col_indices) ||
        (hd.n > 0 && (!modalities || !timestamps || (hd.d > 0 && !embeddings))))
        return set_error(MARS_ERR_INVALID, "null array");
    uint64_t h = mars::fnv1a_update(mars::kFnvOffset, raw, sizeof(raw));
    int rc = mars::read_hashed(f.f, row_offsets, (n + 1) * 4, &h, path);
    if (!rc) rc = mars::read_hashed(f.f, col_indices, uint64_t(hd.e) * 4, &h, path);
    if (!rc) rc = mars::read_hashed(f.f, embeddings, n * uint64_t(hd.d) * 4, &h, path);
    if (!rc) rc = mars::read_hashed(f.f, modalities, n * 4, &h, path);
    if (!rc) rc = mars::read_hashed(f.f, timestamps, n * 4, &h, path);
    uint64_t stored = 0;
    if (!rc) rc = mars::read_hashed(f.f, &stored, sizeof(stored), nullptr, path);
    if (rc) return rc;
    if (stored != h)
        return set_error(MARS_ERR_INVALID, "%s: checksum 0x%016llx, the data hash to 0x%016llx", path,
                         (unsigned long long)stored, (unsigned long long)h);
    return MARS_OK;
}

int mars_kids_file_write(const char* path, int32_t n, int32_t d, const float* embeddings, const float* timestamps,
                         const int32_t* modalities, const int32_t* episode_ids) {
    if (!path || n < 0 || d < 0) return set_error(MARS_ERR_INVALID, "bad arguments");
    if (n > 0 && (!timestamps || !modalities || !episode_ids || (d > 0 && !embeddings)))
        return set_error(MARS_ERR_INVALID, "null array");
    mars::File f;
    f.f = std::fopen(path, "wb");
    if (!f.f) return set_error(MARS_ERR_INVALID, "%s: cannot open for writing", path);
    uint8_t raw[16];
    std::memcpy(raw, &mars::kKidsMagic, 4);
    std::memcpy(raw + 4, &mars::kKidsVersion, 4);
    std::memcpy(raw + 8, &n, 4);
    std::memcpy(raw + 12, &d, 4);
    const uint64_t un = uint64_t(n);
    int rc = mars::write_all(f.f, raw, 16, path);
    if (!rc) rc = mars::write_all(f.f, embeddings, un * uint64_t(d) * 4, path);
    if (!rc) rc = mars::write_all(f.f, timestamps, un * 4, path);
    if (!rc) rc = mars::write_all(f.f, modalities, un * 4, path);
    if (!rc) rc = mars::write_all(f.f, episode_ids, un * 4, path);
    if (rc) return rc;
    const int closed = std::fclose(f.f);
    f.f = nullptr;
    if (closed != 0) return set_error(MARS_ERR_INVALID, "%s: close failed", path);
    return MARS_OK;
}

int mars_kids_file_info(const char* path, int32_t* n, int32_t* d) {
    if (!path || !n || !d) return set_error(MARS_ERR_INVALID, "null argument");
    mars::File f;
    f.f = std::fopen(path, "rb");
    if (!f.f) return set_error(MARS_ERR_INVALID, "%s: cannot open", path);
    return mars::read_kids_header(f.f, path, n, d);
}

int mars_kids_file_read(const char* path, int32_t n, int32_t d, float* embeddings, float* timestamps,
                        int32_t* modalities, int32_t* episode_ids) {
    if (!path) return set_error(MARS_ERR_INVALID, "null path");
    mars::File f;
    f.f = std::fopen(path, "rb");
    if (!f.f) return set_error(MARS_ERR_INVALID, "%s: cannot open", path);
    int32_t fn = 0, fd = 0;
    if (int rc = mars::read_kids_header(f.f, path, &fn, &fd)) return rc;
    if (fn != n || fd != d)
        return set_error(MARS_ERR_INVALID, "%s holds %d x %d (asked %d x %d)", path, fn, fd, n, d);
    if (n > 0 && (!timestamps || !modalities || !episode_ids || (d > 0 && !embeddings)))
        return set_error(MARS_ERR_INVALID, "null array");
    const uint64_t un = uint64_t(n);
    int rc = mars::read_hashed(f.f, embeddings, un * uint64_t(d) * 4, nullptr, path);
    if (!rc) rc = mars::read_hashed(f.f, timestamps, un * 4, nullptr, path);
    if (!rc) rc = mars::read_hashed(f.f, modalities, un * 4, nullptr, path);
    if (!rc) rc = mars::read_hashed(f.f, episode_ids, un * 4, nullptr, path);
    return rc;
}

}  // extern "C"
