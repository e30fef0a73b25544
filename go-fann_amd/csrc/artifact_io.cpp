// artifact_io.cpp -- host readers and writers of the reference's on-disk
// artifacts, so that an index the reference built (graph, sidecars, label
// matrix, query ranges, RaBitQ artifact, DiskANN-style PQ files) loads into
// the views this library searches, and an index built here can be handed
// back.  Plain stdio with 64-bit offsets; every reader validates what the
// reference's loader validates and fails with a message
// (gofann_io_last_error) where the reference throws.
//
// The graph row readers and the PQ code readers take a row window, so a
// caller can stream a file larger than host memory through a pinned staging
// buffer into HBM.
#include <algorithm>
#include <cstdint>
#include <cstdio>
#include <cstring>
#include <limits>
#include <string>
#include <vector>

#include "gofann_hip.h"

namespace {

thread_local std::string g_io_error;

int io_fail(int code, const std::string& msg)
{
    g_io_error = msg;
    return code;
}

struct File {
    FILE* f = nullptr;
    File(const char* path, const char* mode) : f(path ? std::fopen(path, mode) : nullptr) {}
    ~File()
    {
        if (f) std::fclose(f);
    }
    File(const File&) = delete;
    File& operator=(const File&) = delete;
    explicit operator bool() const { return f != nullptr; }
    bool read(void* dst, size_t bytes) { return bytes == 0 || std::fread(dst, 1, bytes, f) == bytes; }
    bool write(const void* src, size_t bytes)
    {
        return bytes == 0 || std::fwrite(src, 1, bytes, f) == bytes;
    }
    bool seek(uint64_t off)
    {
        if (off > static_cast<uint64_t>(std::numeric_limits<off_t>::max())) return false;
        return fseeko(f, static_cast<off_t>(off), SEEK_SET) == 0;
    }
    bool skip(uint64_t bytes)
    {
        if (bytes > static_cast<uint64_t>(std::numeric_limits<off_t>::max())) return false;
        return fseeko(f, static_cast<off_t>(bytes), SEEK_CUR) == 0;
    }
    int64_t size()
    {
        const off_t cur = ftello(f);
        if (cur < 0 || fseeko(f, 0, SEEK_END) != 0) return -1;
        const off_t end = ftello(f);
        if (fseeko(f, cur, SEEK_SET) != 0) return -1;
        return static_cast<int64_t>(end);
    }
    int64_t tell() { return static_cast<int64_t>(ftello(f)); }
    bool close()
    {
        const bool ok = std::fclose(f) == 0;
        f = nullptr;
        return ok;
    }
};

bool mul_ok(uint64_t a, uint64_t b, uint64_t* out)
{
    if (b != 0 && a > std::numeric_limits<uint64_t>::max() / b) return false;
    *out = a * b;
    return true;
}

std::string p(const char* path) { return path ? path : "(null)"; }

// ---------------------------------------------------------------- FDRG graph
// graph_file_format.h:11-25 (header), graph_file_format.cpp (checks, block
// packing: rows never straddle a 4096-byte block; tail of a block is zero).
constexpr uint32_t kGraphMagic = 0x47524446u;  // "FDRG"
constexpr uint32_t kGraphVersion = 1;
constexpr uint32_t kGraphBlock = 4096;
constexpr uint32_t kGraphHeaderBytes = 4096;

static_assert(sizeof(gofann_graph_file_header) == 40, "GraphFileHeader is 40 bytes on disk");

int graph_header_checked(File& in, const char* path, gofann_graph_file_header* h)
{
    if (!in.read(h, sizeof(*h))) return io_fail(GOFANN_ERR_INVALID, "failed to read graph file header from " + p(path));
    if (h->magic != kGraphMagic) return io_fail(GOFANN_ERR_INVALID, "invalid magic in graph file " + p(path));
    if (h->version != kGraphVersion)
        return io_fail(GOFANN_ERR_INVALID, "unsupported graph file version in " + p(path));
    if (h->block_size != kGraphBlock || h->header_size != kGraphHeaderBytes)
        return io_fail(GOFANN_ERR_INVALID, "unexpected block/header size in " + p(path));
    if (h->degree == 0) return io_fail(GOFANN_ERR_INVALID, "degree must be > 0 in " + p(path));
    if (static_cast<uint64_t>(h->row_size_bytes) != static_cast<uint64_t>(h->degree) * 4u)
        return io_fail(GOFANN_ERR_INVALID, "row_size_bytes does not match degree in " + p(path));
    const uint64_t rpb = h->row_size_bytes <= kGraphBlock ? kGraphBlock / h->row_size_bytes : 0;
    if (rpb == 0 || h->rows_per_block != rpb)
        return io_fail(GOFANN_ERR_INVALID, "rows_per_block is invalid in " + p(path));
    uint64_t blocks = h->rows / rpb + (h->rows % rpb ? 1 : 0), payload = 0;
    if (!mul_ok(blocks, kGraphBlock, &payload) ||
        payload > static_cast<uint64_t>(std::numeric_limits<off_t>::max()) - kGraphHeaderBytes)
        return io_fail(GOFANN_ERR_INVALID, "graph file byte count overflows in " + p(path));
    return GOFANN_OK;
}

int graph_header_for(uint64_t rows, uint32_t degree, const char* path, gofann_graph_file_header* h)
{
    if (degree == 0) return io_fail(GOFANN_ERR_INVALID, "degree must be > 0 for graph file output " + p(path));
    if (degree > kGraphBlock / 4u)
        return io_fail(GOFANN_ERR_INVALID, "degree too large for 4KB block packing in " + p(path));
    std::memset(h, 0, sizeof(*h));
    h->magic = kGraphMagic;
    h->version = kGraphVersion;
    h->block_size = kGraphBlock;
    h->header_size = kGraphHeaderBytes;
    h->rows = rows;
    h->degree = degree;
    h->row_size_bytes = degree * 4u;
    h->rows_per_block = kGraphBlock / h->row_size_bytes;
    uint64_t blocks = rows / h->rows_per_block + (rows % h->rows_per_block ? 1 : 0), payload = 0;
    if (!mul_ok(blocks, kGraphBlock, &payload) ||
        payload > static_cast<uint64_t>(std::numeric_limits<off_t>::max()) - kGraphHeaderBytes)
        return io_fail(GOFANN_ERR_INVALID, "graph file byte count overflows for " + p(path));
    return GOFANN_OK;
}

// Packs rows [0, h.rows) into blocks after the header block.  fill(dst, row,
// count) writes `count` consecutive rows starting at `row` to dst; when rows
// tile a block exactly and the source is in memory (`direct` non-null), full
// blocks are written straight from it.
template <typename Fill>
int graph_write_blocks(File& out, const gofann_graph_file_header& h, const char* path,
                       const char* direct, Fill fill)
{
    std::vector<char> block(kGraphHeaderBytes, 0);
    std::memcpy(block.data(), &h, sizeof(h));
    if (!out.write(block.data(), block.size()))
        return io_fail(GOFANN_ERR_INVALID, "failed to write graph file header to " + p(path));
    const uint64_t rpb = h.rows_per_block;
    const uint64_t row_bytes = h.row_size_bytes;
    uint64_t row = 0;
    if (direct && kGraphBlock % row_bytes == 0) {
        row = h.rows / rpb * rpb;
        if (!out.write(direct, row * row_bytes))
            return io_fail(GOFANN_ERR_INVALID, "failed writing packed block to " + p(path));
    }
    // Whole blocks are assembled in a buffer of up to 8 MiB before each write.
    const uint64_t blocks_per_write = 2048;
    std::vector<char> buf(blocks_per_write * kGraphBlock);
    const uint64_t used = rpb * row_bytes;
    while (row < h.rows) {
        uint64_t nb = 0;
        for (; nb < blocks_per_write && row < h.rows; ++nb) {
            const uint64_t in_block = std::min<uint64_t>(rpb, h.rows - row);
            char* dst = buf.data() + nb * kGraphBlock;
            if (!fill(dst, row, in_block))
                return io_fail(GOFANN_ERR_INVALID, "failed reading row payload for " + p(path));
            std::memset(dst + in_block * row_bytes, 0, kGraphBlock - std::min<uint64_t>(used, in_block * row_bytes));
            row += in_block;
        }
        if (!out.write(buf.data(), nb * kGraphBlock))
            return io_fail(GOFANN_ERR_INVALID, "failed writing packed block to " + p(path));
    }
    if (!out.close()) return io_fail(GOFANN_ERR_INVALID, "failed to finish graph file " + p(path));
    return GOFANN_OK;
}

// ------------------------------------------------------- metadata sidecars
// GraphMetadataSidecarHeader (dataloader.h:630-644, version 1) followed by
// cat_freq, group_posting_size, label_size, label_offset [label_count] u32,
// row_to_sample [total_rows] u32, row_filter_mask [total_rows] u64,
// label_filter_bit [original_label_count] u64 (dataloader.cpp:7782-7821).
static_assert(sizeof(gofann_graph_metadata_header) == 88, "metadata sidecar header is 88 bytes");
constexpr uint32_t kMetadataVersion = 1;
// GraphSeedFileHeader (dataloader.h:609-617, version 2) + seed [label_count] u32.
static_assert(sizeof(gofann_graph_seed_header) == 48, "seed sidecar header is 48 bytes");
constexpr uint32_t kSeedVersion = 2;

int metadata_header_checked(File& in, const char* path, gofann_graph_metadata_header* h)
{
    if (!in.read(h, sizeof(*h)))
        return io_fail(GOFANN_ERR_INVALID, "failed to read metadata sidecar header from " + p(path));
    if (h->version != kMetadataVersion)
        return io_fail(GOFANN_ERR_INVALID, "unsupported metadata sidecar version in " + p(path));
    const uint64_t u32max = std::numeric_limits<uint32_t>::max();
    if (h->label_count > u32max || h->original_label_count > u32max || h->total_rows > u32max)
        return io_fail(GOFANN_ERR_INVALID, "metadata sidecar counts exceed uint32 in " + p(path));
    if (h->group_count != h->label_count)
        return io_fail(GOFANN_ERR_INVALID, "metadata sidecar group_count differs from label_count in " + p(path));
    return GOFANN_OK;
}

// ------------------------------------------------------------------- RaBitQ
// RabitqArtifactHeader + RabitqCodecSpec (backend_rabitq.cuh:16-32), then
// eight u64-size-prefixed arrays (backend_rabitq.cu:2748-2845).
struct RabitqDiskHeader {
    uint32_t version, dim, num_anchors, code_bytes;
    uint64_t num_points;
};
struct RabitqDiskCodec {
    uint32_t padded_dim, bits_per_dim, short_code_words, long_code_bytes, layout_flags,
        short_factor_count, ex_factor_count;
};
static_assert(sizeof(RabitqDiskHeader) == 24 && sizeof(RabitqDiskCodec) == 28, "RaBitQ header layout");
constexpr uint32_t kRabitqVersion = 2;
constexpr uint32_t kRabitqMaxBits = 9;
constexpr uint32_t kRabitqLayoutRequired = 1u | 2u | 4u;  // sample-major, MSB-32 short codes, cuVS batch factors
constexpr int kRabitqArrays = 8;

// backend_rabitq.cu:1172-1250 (validate_codec_spec, validate_header).
int rabitq_validate(const gofann_rabitq_file_header& h, const char* path)
{
    if (h.version != kRabitqVersion) return io_fail(GOFANN_ERR_INVALID, "unsupported artifact version in " + p(path));
    if (h.dim == 0 || h.num_anchors == 0 || h.num_points == 0)
        return io_fail(GOFANN_ERR_INVALID, "artifact header contains zero-sized fields in " + p(path));
    if (h.padded_dim < h.dim || h.padded_dim % 64u != 0)
        return io_fail(GOFANN_ERR_INVALID, "artifact codec padded_dim is invalid in " + p(path));
    if (h.bits_per_dim == 0 || h.bits_per_dim > kRabitqMaxBits)
        return io_fail(GOFANN_ERR_INVALID, "artifact codec bits_per_dim is invalid in " + p(path));
    if (h.short_code_words != (h.padded_dim + 31u) / 32u)
        return io_fail(GOFANN_ERR_INVALID, "artifact codec short_code_words is invalid in " + p(path));
    const uint32_t long_bytes =
        h.bits_per_dim <= 1 ? 0u
                            : static_cast<uint32_t>(static_cast<uint64_t>(h.padded_dim) * (h.bits_per_dim - 1u) / 8u);
    if (h.long_code_bytes != long_bytes)
        return io_fail(GOFANN_ERR_INVALID, "artifact codec long_code_bytes is invalid in " + p(path));
    if ((h.layout_flags & kRabitqLayoutRequired) != kRabitqLayoutRequired)
        return io_fail(GOFANN_ERR_INVALID, "artifact codec layout_flags are invalid in " + p(path));
    if (h.short_factor_count != 3 || h.ex_factor_count != 2)
        return io_fail(GOFANN_ERR_INVALID, "artifact codec factor counts are invalid in " + p(path));
    if (h.code_bytes != h.short_code_words * 4u)
        return io_fail(GOFANN_ERR_INVALID, "artifact header code_bytes does not match dim in " + p(path));
    // Bounds that keep every array's byte count inside 64 bits (2^40 points
    // of at most 2^16 bytes per array row).
    if (h.padded_dim > (1u << 16) || h.num_points > (1ull << 40))
        return io_fail(GOFANN_ERR_INVALID, "artifact header sizes are out of range in " + p(path));
    return GOFANN_OK;
}

// Element counts and sizes of the eight arrays, in file order: anchors,
// rotation, query_scaling_factors, anchor_ids, codes, long_codes, factors,
// ex_factors (load_rabitq_index's expected sizes, backend_rabitq.cu:2821-2838).
void rabitq_counts(const gofann_rabitq_file_header& h, uint64_t count[kRabitqArrays], uint32_t elem[kRabitqArrays])
{
    const uint64_t n = h.num_points;
    count[0] = uint64_t(h.num_anchors) * h.padded_dim;
    count[1] = uint64_t(h.padded_dim) * h.padded_dim;
    count[2] = 2;
    count[3] = n;
    count[4] = n * h.code_bytes;
    count[5] = n * h.long_code_bytes;
    count[6] = n * h.short_factor_count;
    count[7] = n * h.ex_factor_count;
    const uint32_t e[kRabitqArrays] = {4, 4, 4, 4, 1, 1, 4, 4};
    std::copy(e, e + kRabitqArrays, elem);
}

int rabitq_open(File& in, const char* path, gofann_rabitq_file_header* h)
{
    if (!in) return io_fail(GOFANN_ERR_INVALID, "unable to open artifact for reading: " + p(path));
    RabitqDiskHeader dh;
    RabitqDiskCodec dc;
    if (!in.read(&dh, sizeof(dh))) return io_fail(GOFANN_ERR_INVALID, "failed to read artifact header from " + p(path));
    if (!in.read(&dc, sizeof(dc))) return io_fail(GOFANN_ERR_INVALID, "failed to read artifact codec spec from " + p(path));
    h->version = dh.version;
    h->dim = dh.dim;
    h->num_anchors = dh.num_anchors;
    h->code_bytes = dh.code_bytes;
    h->num_points = dh.num_points;
    h->padded_dim = dc.padded_dim;
    h->bits_per_dim = dc.bits_per_dim;
    h->short_code_words = dc.short_code_words;
    h->long_code_bytes = dc.long_code_bytes;
    h->layout_flags = dc.layout_flags;
    h->short_factor_count = dc.short_factor_count;
    h->ex_factor_count = dc.ex_factor_count;
    return rabitq_validate(*h, path);
}

// -------------------------------------------------------- DiskANN PQ files
// A "bin" matrix is int32 rows, int32 cols, then rows*cols values
// (load_bin_prefix_local, backend_pq.cu:1716-1747: negative counts read as 0).
struct BinDims {
    uint64_t rows = 0, cols = 0;
};

bool read_bin_dims(File& in, uint64_t offset, BinDims* d)
{
    int32_t r = 0, c = 0;
    if (!in.seek(offset) || !in.read(&r, 4) || !in.read(&c, 4)) return false;
    d->rows = static_cast<uint64_t>(std::max(0, r));
    d->cols = static_cast<uint64_t>(std::max(0, c));
    return true;
}

// The pivot file: offset table (4 or 5 size_t rows, load_pq_pivots_local,
// backend_pq.cu:1767-1795), centres [256][dim] at off[0], mean [dim][1] at
// off[1], chunk boundaries [M+1][1] u32 at off[2] (off[3] in the five-entry
// layout).  Writer: tools/quantization/pq_builder.cu:110-122.
struct Pivots {
    uint64_t off_tables = 0, off_mean = 0, off_chunks = 0;
    uint64_t dim = 0, chunks = 0;  // chunks = M (boundary rows - 1)
};

int pivots_open(File& in, const char* path, Pivots* pv)
{
    if (!in) return io_fail(GOFANN_ERR_INVALID, "unable to open bin file " + p(path));
    BinDims d;
    if (!read_bin_dims(in, 0, &d)) return io_fail(GOFANN_ERR_INVALID, "failed to read bin header from " + p(path));
    if (d.rows != 4 && d.rows != 5) return io_fail(GOFANN_ERR_INVALID, "unexpected pq pivots offset table size in " + p(path));
    uint64_t offs[5] = {};
    if (!in.read(offs, d.rows * d.cols * 8 > 40 ? 40 : d.rows * d.cols * 8))
        return io_fail(GOFANN_ERR_INVALID, "failed to read bin payload from " + p(path));
    pv->off_tables = offs[0];
    pv->off_mean = offs[1];
    pv->off_chunks = d.rows == 5 ? offs[3] : offs[2];
    BinDims t, m, c;
    if (!read_bin_dims(in, pv->off_tables, &t) || !read_bin_dims(in, pv->off_mean, &m) ||
        !read_bin_dims(in, pv->off_chunks, &c))
        return io_fail(GOFANN_ERR_INVALID, "failed to read bin header from " + p(path));
    if (t.rows != 256 || t.cols == 0)
        return io_fail(GOFANN_ERR_INVALID, "pq pivot table is not [256][dim] in " + p(path));
    if (m.rows * m.cols != t.cols)
        return io_fail(GOFANN_ERR_INVALID, "pq pivot mean does not match dim in " + p(path));
    if (c.cols != 1 || c.rows < 2) return io_fail(GOFANN_ERR_INVALID, "unexpected pq chunk offsets shape in " + p(path));
    pv->dim = t.cols;
    pv->chunks = c.rows - 1;
    return GOFANN_OK;
}

}  // namespace

extern "C" {

const char* gofann_io_last_error(void) { return g_io_error.c_str(); }

// ---------------------------------------------------------------- FDRG graph
int gofann_graph_file_has_magic(const char* path)
{
    File in(path, "rb");
    uint32_t magic = 0;
    if (!in || !in.read(&magic, 4)) return io_fail(GOFANN_ERR_INVALID, "unable to read format marker from " + p(path));
    return magic == kGraphMagic ? 1 : 0;
}

int gofann_graph_file_read_header(const char* path, gofann_graph_file_header* out)
{
    if (!out) return io_fail(GOFANN_ERR_INVALID, "null header output");
    File in(path, "rb");
    if (!in) return io_fail(GOFANN_ERR_INVALID, "unable to open graph file " + p(path));
    return graph_header_checked(in, path, out);
}

int gofann_graph_file_read_rows(const char* path, uint64_t row_begin, uint64_t row_count, uint32_t* out)
{
    File in(path, "rb");
    if (!in) return io_fail(GOFANN_ERR_INVALID, "unable to open graph file " + p(path));
    gofann_graph_file_header h;
    int rc = graph_header_checked(in, path, &h);
    if (rc != GOFANN_OK) return rc;
    if (row_begin > h.rows || row_count > h.rows - row_begin)
        return io_fail(GOFANN_ERR_INVALID, "row window exceeds the graph file's rows in " + p(path));
    if (row_count == 0) return GOFANN_OK;
    if (!out) return io_fail(GOFANN_ERR_INVALID, "null row output");
    const uint64_t rpb = h.rows_per_block;
    // The reference reads whole blocks, so a file whose last needed block is
    // short is an error, not a partial read.
    const uint64_t last_block = (row_begin + row_count - 1) / rpb;
    const int64_t size = in.size();
    if (size < 0 || static_cast<uint64_t>(size) < kGraphHeaderBytes + (last_block + 1) * kGraphBlock)
        return io_fail(GOFANN_ERR_INVALID, "failed reading graph file block from " + p(path));
    const size_t row_bytes = h.row_size_bytes;
    if (kGraphBlock % row_bytes == 0) {
        // Rows tile the blocks exactly: the payload is the row-major matrix.
        if (!in.seek(kGraphHeaderBytes + row_begin * row_bytes) || !in.read(out, row_count * row_bytes))
            return io_fail(GOFANN_ERR_INVALID, "failed reading graph file block from " + p(path));
        return GOFANN_OK;
    }
    const uint64_t blocks_per_read = 2048;
    std::vector<char> buf(blocks_per_read * kGraphBlock);
    uint64_t row = row_begin;
    const uint64_t end = row_begin + row_count;
    char* dst = reinterpret_cast<char*>(out);
    while (row < end) {
        const uint64_t b0 = row / rpb;
        const uint64_t nb = std::min<uint64_t>(blocks_per_read, last_block + 1 - b0);
        if (!in.seek(kGraphHeaderBytes + b0 * kGraphBlock) || !in.read(buf.data(), nb * kGraphBlock))
            return io_fail(GOFANN_ERR_INVALID, "failed reading graph file block from " + p(path));
        const uint64_t stop = std::min<uint64_t>(end, (b0 + nb) * rpb);
        for (; row < stop; ++row) {
            const uint64_t b = row / rpb - b0, r = row % rpb;
            std::memcpy(dst, buf.data() + b * kGraphBlock + r * row_bytes, row_bytes);
            dst += row_bytes;
        }
    }
    return GOFANN_OK;
}

int gofann_graph_file_write(const char* path, const uint32_t* rows, uint64_t row_count, uint32_t degree)
{
    gofann_graph_file_header h;
    int rc = graph_header_for(row_count, degree, path, &h);
    if (rc != GOFANN_OK) return rc;
    if (row_count && !rows) return io_fail(GOFANN_ERR_INVALID, "null rows for graph file output " + p(path));
    File out(path, "wb");
    if (!out) return io_fail(GOFANN_ERR_INVALID, "unable to open graph file output " + p(path));
    const char* src = reinterpret_cast<const char*>(rows);
    return graph_write_blocks(out, h, path, src, [&](char* dst, uint64_t row, uint64_t count) {
        std::memcpy(dst, src + row * h.row_size_bytes, count * h.row_size_bytes);
        return true;
    });
}

int gofann_graph_file_convert_legacy(const char* legacy_path, const char* path)
{
    File in(legacy_path, "rb");
    if (!in) return io_fail(GOFANN_ERR_INVALID, "unable to open legacy graph " + p(legacy_path));
    uint64_t rows = 0, cols = 0;
    if (!in.read(&rows, 8) || !in.read(&cols, 8))
        return io_fail(GOFANN_ERR_INVALID, "failed to read legacy graph header from " + p(legacy_path));
    if (cols == 0 || cols > std::numeric_limits<uint32_t>::max())
        return io_fail(GOFANN_ERR_INVALID, "invalid degree in legacy graph " + p(legacy_path));
    gofann_graph_file_header h;
    int rc = graph_header_for(rows, static_cast<uint32_t>(cols), path, &h);
    if (rc != GOFANN_OK) return rc;
    File out(path, "wb");
    if (!out) return io_fail(GOFANN_ERR_INVALID, "unable to open graph file output " + p(path));
    return graph_write_blocks(out, h, path, nullptr, [&](char* dst, uint64_t, uint64_t count) {
        return in.read(dst, count * h.row_size_bytes);
    });
}

// ------------------------------------------------------- metadata sidecars
int gofann_graph_metadata_read_header(const char* path, gofann_graph_metadata_header* out)
{
    if (!out) return io_fail(GOFANN_ERR_INVALID, "null header output");
    File in(path, "rb");
    if (!in) return io_fail(GOFANN_ERR_INVALID, "unable to open metadata sidecar " + p(path));
    return metadata_header_checked(in, path, out);
}

int gofann_graph_metadata_read(const char* path, uint32_t* cat_freq, uint32_t* group_posting_size,
                               uint32_t* label_size, uint32_t* label_offset, uint32_t* row_to_sample,
                               uint64_t* row_filter_mask, uint64_t* label_filter_bit)
{
    File in(path, "rb");
    if (!in) return io_fail(GOFANN_ERR_INVALID, "unable to open metadata sidecar " + p(path));
    gofann_graph_metadata_header h;
    int rc = metadata_header_checked(in, path, &h);
    if (rc != GOFANN_OK) return rc;
    const uint64_t L = h.label_count, R = h.total_rows, O = h.original_label_count;
    std::vector<uint32_t> cf(L), gp(L), ls(L), lo(L), rs(R);
    if (!in.read(cf.data(), L * 4) || !in.read(gp.data(), L * 4) || !in.read(ls.data(), L * 4) ||
        !in.read(lo.data(), L * 4) || !in.read(rs.data(), R * 4))
        return io_fail(GOFANN_ERR_INVALID, "metadata sidecar ended early: " + p(path));
    // validate_metadata_sidecar_vectors (dataloader.cpp:7612-7690), the part
    // that does not need the group layout.
    uint64_t expected = 0;
    for (uint64_t g = 0; g < L; ++g) {
        if (cf[g] != gp[g]) return io_fail(GOFANN_ERR_INVALID, "cat_freq/group_posting_size mismatch in " + p(path));
        if (lo[g] != expected) return io_fail(GOFANN_ERR_INVALID, "label_offset is not contiguous in " + p(path));
        expected += ls[g];
        if (ls[g] > 0 && cf[g] <= static_cast<uint32_t>(static_cast<int>(h.specificity_threshold)))
            return io_fail(GOFANN_ERR_INVALID,
                           "high-frequency label_size conflicts with specificity_threshold in " + p(path));
    }
    if (expected != R) return io_fail(GOFANN_ERR_INVALID, "label_size sum does not match total_rows in " + p(path));
    for (uint64_t r = 0; r < R; ++r)
        if (rs[r] >= h.num_points) return io_fail(GOFANN_ERR_INVALID, "row_to_sample exceeds num_points in " + p(path));
    if (row_filter_mask) {
        if (!in.read(row_filter_mask, R * 8))
            return io_fail(GOFANN_ERR_INVALID, "metadata sidecar ended while reading row_filter_mask: " + p(path));
    } else if (!in.skip(R * 8)) {
        return io_fail(GOFANN_ERR_INVALID, "metadata sidecar ended while reading row_filter_mask: " + p(path));
    }
    std::vector<uint64_t> lfb(O);
    if (!in.read(lfb.data(), O * 8))
        return io_fail(GOFANN_ERR_INVALID, "metadata sidecar ended while reading label_filter_bit: " + p(path));
    auto put = [](uint32_t* dst, const std::vector<uint32_t>& v) {
        if (dst && !v.empty()) std::memcpy(dst, v.data(), v.size() * 4);
    };
    put(cat_freq, cf);
    put(group_posting_size, gp);
    put(label_size, ls);
    put(label_offset, lo);
    put(row_to_sample, rs);
    if (label_filter_bit && O) std::memcpy(label_filter_bit, lfb.data(), O * 8);
    return GOFANN_OK;
}

int gofann_graph_metadata_write(const char* path, const gofann_graph_metadata_header* header,
                                const uint32_t* cat_freq, const uint32_t* group_posting_size,
                                const uint32_t* label_size, const uint32_t* label_offset,
                                const uint32_t* row_to_sample, const uint64_t* row_filter_mask,
                                const uint64_t* label_filter_bit)
{
    if (!header) return io_fail(GOFANN_ERR_INVALID, "null metadata header");
    gofann_graph_metadata_header h = *header;
    h.version = kMetadataVersion;
    h.reserved = 0;
    const uint64_t L = h.label_count, R = h.total_rows, O = h.original_label_count;
    if ((L && (!cat_freq || !group_posting_size || !label_size || !label_offset)) || (R && !row_to_sample) ||
        (O && !label_filter_bit))
        return io_fail(GOFANN_ERR_INVALID, "null metadata array");
    File out(path, "wb");
    if (!out) return io_fail(GOFANN_ERR_INVALID, "unable to write metadata sidecar " + p(path));
    bool ok = out.write(&h, sizeof(h)) && out.write(cat_freq, L * 4) && out.write(group_posting_size, L * 4) &&
              out.write(label_size, L * 4) && out.write(label_offset, L * 4) && out.write(row_to_sample, R * 4);
    if (ok) {
        if (row_filter_mask) {
            ok = out.write(row_filter_mask, R * 8);
        } else {
            // The all-ones mask of an ungrouped layout (one label per group).
            const std::vector<uint64_t> ones(std::min<uint64_t>(R, 1u << 16), ~0ull);
            for (uint64_t r = 0; ok && r < R; r += ones.size())
                ok = out.write(ones.data(), std::min<uint64_t>(ones.size(), R - r) * 8);
        }
    }
    ok = ok && out.write(label_filter_bit, O * 8) && out.close();
    if (!ok) return io_fail(GOFANN_ERR_INVALID, "failed to write metadata sidecar " + p(path));
    return GOFANN_OK;
}

// group_layout_checksum (dataloader.cpp:320-332): FNV-1a over the little-
// endian bytes of (groups, labels, then per group its size and labels).
uint64_t gofann_group_layout_checksum(const uint32_t* group_offsets, const uint32_t* group_labels,
                                      uint32_t groups, uint32_t label_count)
{
    uint64_t hash = 1469598103934665603ull;
    auto mix = [&](uint64_t v) {
        for (int b = 0; b < 8; ++b) {
            hash ^= (v >> (8 * b)) & 0xffu;
            hash *= 1099511628211ull;
        }
    };
    mix(groups);
    mix(label_count);
    for (uint32_t g = 0; g < groups; ++g) {
        const uint32_t b = group_offsets ? group_offsets[g] : g;
        const uint32_t e = group_offsets ? group_offsets[g + 1] : g + 1;
        mix(e - b);
        for (uint32_t i = b; i < e; ++i) mix(group_labels ? group_labels[i] : i);
    }
    return hash;
}

int gofann_graph_seeds_read_header(const char* path, gofann_graph_seed_header* out)
{
    if (!out) return io_fail(GOFANN_ERR_INVALID, "null header output");
    File in(path, "rb");
    if (!in) return io_fail(GOFANN_ERR_INVALID, "unable to open seed sidecar " + p(path));
    if (!in.read(out, sizeof(*out))) return io_fail(GOFANN_ERR_INVALID, "failed to read seed sidecar header from " + p(path));
    if (out->version != kSeedVersion) return io_fail(GOFANN_ERR_INVALID, "unsupported seed sidecar version in " + p(path));
    if (out->label_count > std::numeric_limits<uint32_t>::max())
        return io_fail(GOFANN_ERR_INVALID, "seed sidecar label count exceeds uint32 in " + p(path));
    return GOFANN_OK;
}

int gofann_graph_seeds_read(const char* path, const uint32_t* label_size, uint32_t* seeds)
{
    gofann_graph_seed_header h;
    int rc = gofann_graph_seeds_read_header(path, &h);
    if (rc != GOFANN_OK) return rc;
    File in(path, "rb");
    if (!in || !in.seek(sizeof(h))) return io_fail(GOFANN_ERR_INVALID, "unable to open seed sidecar " + p(path));
    std::vector<uint32_t> s(h.label_count);
    if (!in.read(s.data(), s.size() * 4)) return io_fail(GOFANN_ERR_INVALID, "seed sidecar ended early: " + p(path));
    // load_seed_sidecar (dataloader.cpp:7538-7550): an empty label has no
    // seed; any other label's seed is a label-local row id.
    if (label_size) {
        for (uint64_t l = 0; l < h.label_count; ++l) {
            const bool ok = label_size[l] == 0 ? s[l] == UINT32_MAX : s[l] != UINT32_MAX && s[l] < label_size[l];
            if (!ok) return io_fail(GOFANN_ERR_INVALID, "seed sidecar seed is invalid for label " + std::to_string(l));
        }
    }
    if (seeds && !s.empty()) std::memcpy(seeds, s.data(), s.size() * 4);
    return GOFANN_OK;
}

int gofann_graph_seeds_write(const char* path, const gofann_graph_seed_header* header, const uint32_t* seeds)
{
    if (!header) return io_fail(GOFANN_ERR_INVALID, "null seed header");
    gofann_graph_seed_header h = *header;
    h.version = kSeedVersion;
    h.reserved = 0;
    if (h.label_count && !seeds) return io_fail(GOFANN_ERR_INVALID, "null seeds");
    File out(path, "wb");
    if (!out || !out.write(&h, sizeof(h)) || !out.write(seeds, h.label_count * 4) || !out.close())
        return io_fail(GOFANN_ERR_INVALID, "failed to write seed sidecar " + p(path));
    return GOFANN_OK;
}

// ------------------------------------------------------------------- spmat
// u64 rows, cols, nnz; u64 indptr[rows + 1]; u32 indices[nnz]
// (load_spmat_labels, dataloader.cpp:6663-6760).
int gofann_spmat_read_header(const char* path, uint64_t* rows, uint64_t* cols, uint64_t* nnz)
{
    File in(path, "rb");
    if (!in) return io_fail(GOFANN_ERR_INVALID, "unable to open spmat label file " + p(path));
    uint64_t h[3];
    if (!in.read(h, sizeof(h))) return io_fail(GOFANN_ERR_INVALID, "invalid spmat header in " + p(path));
    if (h[0] > std::numeric_limits<uint32_t>::max())
        return io_fail(GOFANN_ERR_INVALID, "spmat row count exceeds uint32 range in " + p(path));
    if (h[1] > std::numeric_limits<uint32_t>::max())
        return io_fail(GOFANN_ERR_INVALID, "spmat label count exceeds uint32 range in " + p(path));
    if (rows) *rows = h[0];
    if (cols) *cols = h[1];
    if (nnz) *nnz = h[2];
    return GOFANN_OK;
}

int gofann_spmat_read(const char* path, uint32_t row_limit, uint64_t* indptr, uint32_t* indices,
                      uint64_t capacity, uint64_t* out_nnz)
{
    uint64_t rows = 0, cols = 0, nnz = 0;
    int rc = gofann_spmat_read_header(path, &rows, &cols, &nnz);
    if (rc != GOFANN_OK) return rc;
    const uint64_t eff = (row_limit > 0 && row_limit < rows) ? row_limit : rows;
    if (!indptr) return io_fail(GOFANN_ERR_INVALID, "null spmat indptr output");
    File in(path, "rb");
    if (!in || !in.seek(24) || !in.read(indptr, (eff + 1) * 8))
        return io_fail(GOFANN_ERR_INVALID, "failed to read spmat indptr from " + p(path));
    if (indptr[0] != 0) return io_fail(GOFANN_ERR_INVALID, "spmat indptr must start at 0 in " + p(path));
    for (uint64_t r = 0; r < eff; ++r) {
        if (indptr[r] > indptr[r + 1]) return io_fail(GOFANN_ERR_INVALID, "spmat indptr is not monotonic in " + p(path));
        if (indptr[r + 1] > nnz) return io_fail(GOFANN_ERR_INVALID, "spmat indptr exceeds nnz in " + p(path));
    }
    const uint64_t raw = indptr[eff];
    if (raw > capacity || (raw && !indices))
        return io_fail(GOFANN_ERR_INVALID, "spmat index capacity is short for " + p(path));
    if (!in.seek(24 + (rows + 1) * 8) || !in.read(indices, raw * 4))
        return io_fail(GOFANN_ERR_INVALID, "failed to read spmat indices from " + p(path));
    // Each row's labels sorted and de-duplicated, rows compacted in place.
    uint64_t w = 0;
    for (uint64_t r = 0; r < eff; ++r) {
        const uint64_t b = indptr[r], e = indptr[r + 1];
        indptr[r] = w;
        uint32_t* rb = indices + b;
        uint32_t* re = indices + e;
        for (uint32_t* it = rb; it != re; ++it)
            if (*it >= cols) return io_fail(GOFANN_ERR_INVALID, "spmat label index out of range in " + p(path));
        std::sort(rb, re);
        const uint64_t n = static_cast<uint64_t>(std::unique(rb, re) - rb);
        if (w != b && n) std::memmove(indices + w, rb, n * 4);
        w += n;
    }
    indptr[eff] = w;
    if (out_nnz) *out_nnz = w;
    return GOFANN_OK;
}

// ------------------------------------------------------------ query ranges
// u32 query_count, then per query a record {u8 mode, f32 upper, f32 lower}
// packed (9 bytes) or aligned (12 bytes); or u32 query_count, u32
// range_count and query_count * range_count records of either form
// (load_query_range_binary, dataloader.cpp:6780-6880).
int gofann_query_range_read_header(const char* path, uint32_t expected_queries, uint32_t* range_count,
                                   uint32_t* record_bytes)
{
    if (!path || !*path) {
        if (range_count) *range_count = 1;
        if (record_bytes) *record_bytes = 0;
        return GOFANN_OK;
    }
    File in(path, "rb");
    if (!in) return io_fail(GOFANN_ERR_INVALID, "unable to open query range file " + p(path));
    uint32_t q = 0;
    if (!in.read(&q, 4)) return io_fail(GOFANN_ERR_INVALID, "invalid query range header in " + p(path));
    if (q != expected_queries) return io_fail(GOFANN_ERR_INVALID, "query range count does not match query vector rows");
    const int64_t size = in.size();
    if (size < 4) return io_fail(GOFANN_ERR_INVALID, "invalid query range header in " + p(path));
    const uint64_t payload = static_cast<uint64_t>(size) - 4;
    uint32_t rc = 1, rec = 0;
    if (payload == uint64_t(q) * 12) {
        rec = 12;
    } else if (payload == uint64_t(q) * 9) {
        rec = 9;
    } else {
        if (!in.read(&rc, 4) || rc == 0)
            return io_fail(GOFANN_ERR_INVALID, "query range payload size does not match packed/aligned layouts for " + p(path));
        const uint64_t merged = payload - 4;
        if (merged == uint64_t(q) * rc * 12) {
            rec = 12;
        } else if (merged == uint64_t(q) * rc * 9) {
            rec = 9;
        } else {
            return io_fail(GOFANN_ERR_INVALID, "query range payload size does not match packed/aligned layouts for " + p(path));
        }
    }
    if (range_count) *range_count = rc;
    if (record_bytes) *record_bytes = rec;
    return GOFANN_OK;
}

int gofann_query_range_read(const char* path, uint32_t expected_queries, uint8_t* modes, float* lower, float* upper)
{
    uint32_t rc = 0, rec = 0;
    int st = gofann_query_range_read_header(path, expected_queries, &rc, &rec);
    if (st != GOFANN_OK) return st;
    const uint64_t total = uint64_t(expected_queries) * rc;
    if (total && (!modes || !lower || !upper)) return io_fail(GOFANN_ERR_INVALID, "null query range output");
    if (rec == 0) {
        // No file: one unconstrained range per query.
        std::memset(modes, 0, total);
        std::memset(lower, 0, total * 4);
        std::memset(upper, 0, total * 4);
        return GOFANN_OK;
    }
    File in(path, "rb");
    std::vector<uint8_t> buf(total * rec);
    if (!in) return io_fail(GOFANN_ERR_INVALID, "unable to open query range file " + p(path));
    // The records end the file: they start after query_count, or after
    // query_count and range_count in the multi-range layout.
    const int64_t size = in.size();
    const uint64_t start = static_cast<uint64_t>(size) - total * rec;
    if (!in.seek(start) || !in.read(buf.data(), buf.size()))
        return io_fail(GOFANN_ERR_INVALID, "failed to read query range payload from " + p(path));
    for (uint64_t i = 0; i < total; ++i) {
        const uint8_t* r = buf.data() + i * rec;
        const size_t fo = rec == 12 ? 4 : 1;
        modes[i] = r[0];
        std::memcpy(&upper[i], r + fo, 4);
        std::memcpy(&lower[i], r + fo + 4, 4);
    }
    return GOFANN_OK;
}

// ------------------------------------------------------------------- RaBitQ
int gofann_rabitq_file_read_header(const char* path, gofann_rabitq_file_header* out)
{
    if (!out) return io_fail(GOFANN_ERR_INVALID, "null header output");
    File in(path, "rb");
    int rc = rabitq_open(in, path, out);
    if (rc != GOFANN_OK) return rc;
    // Walk the size prefixes: every array must have the size the header implies.
    uint64_t count[kRabitqArrays];
    uint32_t elem[kRabitqArrays];
    rabitq_counts(*out, count, elem);
    for (int a = 0; a < kRabitqArrays; ++a) {
        uint64_t n = 0;
        if (!in.read(&n, 8)) return io_fail(GOFANN_ERR_INVALID, "failed to read artifact payload from " + p(path));
        if (n != count[a]) return io_fail(GOFANN_ERR_INVALID, "artifact payload sizes do not match header in " + p(path));
        if (!in.skip(n * elem[a])) return io_fail(GOFANN_ERR_INVALID, "failed to read artifact payload from " + p(path));
    }
    const int64_t size = in.size();
    if (size < 0 || in.tell() > size) return io_fail(GOFANN_ERR_INVALID, "failed to read artifact payload from " + p(path));
    return GOFANN_OK;
}

int gofann_rabitq_file_read(const char* path, float* anchors, float* rotation, float* query_scaling_factors,
                            uint32_t* anchor_ids, uint8_t* codes, uint8_t* long_codes, float* factors,
                            float* ex_factors)
{
    gofann_rabitq_file_header h;
    int rc = gofann_rabitq_file_read_header(path, &h);
    if (rc != GOFANN_OK) return rc;
    File in(path, "rb");
    if (!in || !in.seek(sizeof(RabitqDiskHeader) + sizeof(RabitqDiskCodec)))
        return io_fail(GOFANN_ERR_INVALID, "unable to open artifact for reading: " + p(path));
    void* dst[kRabitqArrays] = {anchors, rotation, query_scaling_factors, anchor_ids,
                                codes, long_codes, factors, ex_factors};
    uint64_t count[kRabitqArrays];
    uint32_t elem[kRabitqArrays];
    rabitq_counts(h, count, elem);
    for (int a = 0; a < kRabitqArrays; ++a) {
        uint64_t n = 0;
        if (!in.read(&n, 8)) return io_fail(GOFANN_ERR_INVALID, "failed to read artifact payload from " + p(path));
        // the outputs are sized from the header: the file must still agree
        if (n != count[a]) return io_fail(GOFANN_ERR_INVALID, "artifact payload sizes do not match header in " + p(path));
        if (a == 3) {
            // anchor ids are checked whether or not the caller wants them.
            std::vector<uint32_t> chunk(std::min<uint64_t>(n, 1u << 20));
            uint32_t* out = anchor_ids;
            for (uint64_t i = 0; i < n;) {
                const uint64_t c = std::min<uint64_t>(chunk.size(), n - i);
                uint32_t* buf = out ? out + i : chunk.data();
                if (!in.read(buf, c * 4)) return io_fail(GOFANN_ERR_INVALID, "failed to read artifact payload from " + p(path));
                for (uint64_t j = 0; j < c; ++j)
                    if (buf[j] >= h.num_anchors)
                        return io_fail(GOFANN_ERR_INVALID, "artifact anchor_ids contain an out-of-range anchor id in " + p(path));
                i += c;
            }
            continue;
        }
        if (dst[a]) {
            if (!in.read(dst[a], n * elem[a])) return io_fail(GOFANN_ERR_INVALID, "failed to read artifact payload from " + p(path));
        } else if (!in.skip(n * elem[a])) {
            return io_fail(GOFANN_ERR_INVALID, "failed to read artifact payload from " + p(path));
        }
    }
    return GOFANN_OK;
}

int gofann_rabitq_file_write(const char* path, const gofann_rabitq_file_header* header, const float* anchors,
                             const float* rotation, const float* query_scaling_factors,
                             const uint32_t* anchor_ids, const uint8_t* codes, const uint8_t* long_codes,
                             const float* factors, const float* ex_factors)
{
    if (!header) return io_fail(GOFANN_ERR_INVALID, "null artifact header");
    int rc = rabitq_validate(*header, path);
    if (rc != GOFANN_OK) return rc;
    const gofann_rabitq_file_header& h = *header;
    const void* src[kRabitqArrays] = {anchors, rotation, query_scaling_factors, anchor_ids,
                                      codes, long_codes, factors, ex_factors};
    uint64_t count[kRabitqArrays];
    uint32_t elem[kRabitqArrays];
    rabitq_counts(h, count, elem);
    if (!anchors || !anchor_ids || !codes || !factors || (count[5] && !long_codes))
        return io_fail(GOFANN_ERR_INVALID, "null artifact array");
    for (uint64_t i = 0; i < h.num_points; ++i)
        if (anchor_ids[i] >= h.num_anchors) return io_fail(GOFANN_ERR_INVALID, "artifact anchor_ids contain an out-of-range anchor id");
    File out(path, "wb");
    if (!out) return io_fail(GOFANN_ERR_INVALID, "unable to open artifact for writing: " + p(path));
    const RabitqDiskHeader dh{h.version, h.dim, h.num_anchors, h.code_bytes, h.num_points};
    const RabitqDiskCodec dc{h.padded_dim, h.bits_per_dim, h.short_code_words, h.long_code_bytes,
                             h.layout_flags, h.short_factor_count, h.ex_factor_count};
    bool ok = out.write(&dh, sizeof(dh)) && out.write(&dc, sizeof(dc));
    const std::vector<char> zeros(1 << 16, 0);
    for (int a = 0; ok && a < kRabitqArrays; ++a) {
        ok = out.write(&count[a], 8);
        const uint64_t bytes = count[a] * elem[a];
        if (src[a]) {
            ok = ok && out.write(src[a], bytes);
        } else {
            // Absent rotation rows, scaling factors and ex factors are zeros.
            for (uint64_t b = 0; ok && b < bytes; b += zeros.size())
                ok = out.write(zeros.data(), std::min<uint64_t>(zeros.size(), bytes - b));
        }
    }
    if (!ok || !out.close()) return io_fail(GOFANN_ERR_INVALID, "failed while writing artifact " + p(path));
    return GOFANN_OK;
}

// -------------------------------------------------------- DiskANN PQ files
int gofann_pq_pivots_read_header(const char* path, uint32_t* dim, uint32_t* pq_dim)
{
    File in(path, "rb");
    Pivots pv;
    int rc = pivots_open(in, path, &pv);
    if (rc != GOFANN_OK) return rc;
    if (dim) *dim = static_cast<uint32_t>(pv.dim);
    if (pq_dim) *pq_dim = static_cast<uint32_t>(pv.chunks);
    return GOFANN_OK;
}

int gofann_pq_pivots_read(const char* path, uint32_t pq_dim, float* centroids)
{
    File in(path, "rb");
    Pivots pv;
    int rc = pivots_open(in, path, &pv);
    if (rc != GOFANN_OK) return rc;
    if (pq_dim != 0 && pv.chunks != pq_dim) return io_fail(GOFANN_ERR_INVALID, "unexpected pq chunk offsets shape in " + p(path));
    const uint64_t D = pv.dim, M = pv.chunks;
    std::vector<float> table(256 * D), mean(D);
    std::vector<uint32_t> bounds(M + 1);
    if (!in.seek(pv.off_tables + 8) || !in.read(table.data(), table.size() * 4) || !in.seek(pv.off_mean + 8) ||
        !in.read(mean.data(), D * 4) || !in.seek(pv.off_chunks + 8) || !in.read(bounds.data(), (M + 1) * 4))
        return io_fail(GOFANN_ERR_INVALID, "failed to read bin payload from " + p(path));
    // The kernels split dim into M equal sub-vectors.
    if (M == 0 || D % M != 0) return io_fail(GOFANN_ERR_UNSUPPORTED, "pq dim is not a multiple of the chunk count in " + p(path));
    for (uint64_t m = 0; m <= M; ++m)
        if (bounds[m] != m * (D / M))
            return io_fail(GOFANN_ERR_UNSUPPORTED, "pq chunk boundaries are not uniform in " + p(path));
    if (!centroids) return io_fail(GOFANN_ERR_INVALID, "null centroid output");
    // load_pq_index (backend_pq.cu:1818-1821): centre + mean, one f32 add.
    for (uint64_t i = 0; i < 256 * D; ++i) centroids[i] = table[i] + mean[i % D];
    return GOFANN_OK;
}

int gofann_pq_codes_read_header(const char* path, uint64_t* rows, uint32_t* pq_dim)
{
    File in(path, "rb");
    if (!in) return io_fail(GOFANN_ERR_INVALID, "unable to open bin file " + p(path));
    BinDims d;
    if (!read_bin_dims(in, 0, &d)) return io_fail(GOFANN_ERR_INVALID, "failed to read bin header from " + p(path));
    if (rows) *rows = d.rows;
    if (pq_dim) *pq_dim = static_cast<uint32_t>(d.cols);
    return GOFANN_OK;
}

int gofann_pq_codes_read(const char* path, uint64_t row_begin, uint64_t row_count, uint8_t* out, uint32_t out_stride)
{
    File in(path, "rb");
    if (!in) return io_fail(GOFANN_ERR_INVALID, "unable to open bin file " + p(path));
    BinDims d;
    if (!read_bin_dims(in, 0, &d)) return io_fail(GOFANN_ERR_INVALID, "failed to read bin header from " + p(path));
    if (row_begin > d.rows || row_count > d.rows - row_begin)
        return io_fail(GOFANN_ERR_INVALID, "row window exceeds the code file's rows in " + p(path));
    const uint64_t stride = out_stride ? out_stride : d.cols;
    if (stride < d.cols) return io_fail(GOFANN_ERR_INVALID, "code output stride is shorter than pq_dim");
    if (row_count && !out) return io_fail(GOFANN_ERR_INVALID, "null code output");
    if (!in.seek(8 + row_begin * d.cols)) return io_fail(GOFANN_ERR_INVALID, "failed to read bin payload from " + p(path));
    if (stride == d.cols) {
        if (!in.read(out, row_count * d.cols)) return io_fail(GOFANN_ERR_INVALID, "failed to read bin payload from " + p(path));
        return GOFANN_OK;
    }
    // Codes placed inside wider per-sample records.
    std::vector<uint8_t> buf(std::min<uint64_t>(row_count, 1u << 16) * d.cols);
    for (uint64_t r = 0; r < row_count;) {
        const uint64_t c = std::min<uint64_t>(buf.size() / std::max<uint64_t>(d.cols, 1), row_count - r);
        if (!in.read(buf.data(), c * d.cols)) return io_fail(GOFANN_ERR_INVALID, "failed to read bin payload from " + p(path));
        for (uint64_t j = 0; j < c; ++j) std::memcpy(out + (r + j) * stride, buf.data() + j * d.cols, d.cols);
        r += c;
    }
    return GOFANN_OK;
}

int gofann_pq_files_write(const char* pivots_path, const char* codes_path, const float* centroids, uint32_t dim,
                          uint32_t pq_dim, const uint8_t* codes, uint64_t rows)
{
    if (dim == 0 || pq_dim == 0 || dim % pq_dim != 0)
        return io_fail(GOFANN_ERR_INVALID, "PQ requires dim divisible by pq-dim");
    if (rows > static_cast<uint64_t>(std::numeric_limits<int32_t>::max()) || dim > static_cast<uint32_t>(std::numeric_limits<int32_t>::max()))
        return io_fail(GOFANN_ERR_INVALID, "PQ matrix dimensions exceed int32 format");
    if (!centroids || (rows && !codes)) return io_fail(GOFANN_ERR_INVALID, "null PQ array");
    // Offset table, [256][dim] centres, [dim][1] zero mean, [M+1][1]
    // boundaries (tools/quantization/pq_builder.cu:110-122).
    const uint64_t table_bytes = 256ull * dim * 4;
    const uint64_t first = 8 + 4 * 8;
    uint64_t offs[4] = {first, first + 8 + table_bytes, first + 16 + table_bytes + uint64_t(dim) * 4, 0};
    offs[3] = offs[2] + 8 + (uint64_t(pq_dim) + 1) * 4;
    const std::vector<float> mean(dim, 0.0f);
    std::vector<uint32_t> bounds(pq_dim + 1);
    for (uint32_t i = 0; i <= pq_dim; ++i) bounds[i] = i * (dim / pq_dim);
    auto dims = [](File& f, uint32_t r, uint32_t c) { return f.write(&r, 4) && f.write(&c, 4); };
    File pv(pivots_path, "wb");
    if (!pv) return io_fail(GOFANN_ERR_INVALID, "unable to open output file " + p(pivots_path));
    bool ok = dims(pv, 4, 1) && pv.write(offs, sizeof(offs)) && dims(pv, 256, dim) &&
              pv.write(centroids, table_bytes) && dims(pv, dim, 1) && pv.write(mean.data(), dim * 4u) &&
              dims(pv, pq_dim + 1, 1) && pv.write(bounds.data(), bounds.size() * 4) && pv.close();
    if (!ok) return io_fail(GOFANN_ERR_INVALID, "output write failed: " + p(pivots_path));
    File cf(codes_path, "wb");
    if (!cf) return io_fail(GOFANN_ERR_INVALID, "unable to open output file " + p(codes_path));
    ok = dims(cf, static_cast<uint32_t>(rows), pq_dim) && cf.write(codes, rows * pq_dim) && cf.close();
    if (!ok) return io_fail(GOFANN_ERR_INVALID, "output write failed: " + p(codes_path));
    return GOFANN_OK;
}

}  // extern "C"
