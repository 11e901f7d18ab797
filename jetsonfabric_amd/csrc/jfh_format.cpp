// JFM v2 reader/writer, GGUF metadata and SHA-256 (FIPS 180-4).
// Byte contract: docs/jfm-v2-format.md:18-90, runtime/engines/native/src/format.h:6-36.
#include "jfh_format.hpp"

#include <algorithm>
#include <cerrno>
#include <cstring>
#include <fcntl.h>
#include <filesystem>
#include <fstream>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

namespace jfh {
namespace {

constexpr uint32_t kFormatVersion = 2;
constexpr size_t kManifestHeader = 64;
constexpr size_t kManifestRecord = 72;
constexpr size_t kSegmentHeader = 64;
constexpr size_t kTensorRecord = 80;
constexpr uint64_t kAlign = 64;
constexpr uint32_t kMaxLayers = 4096;
constexpr uint64_t kMaxTensors = 1000000;
constexpr size_t kMaxManifest = 16u << 20;

enum SegmentKind : uint32_t { kShared = 0, kInput = 1, kLayer = 2, kOutput = 3, kMetadata = 4 };

// ---------------------------------------------------------------- SHA-256
struct Sha256 {
    uint32_t h[8] = {0x6a09e667u, 0xbb67ae85u, 0x3c6ef372u, 0xa54ff53au,
                     0x510e527fu, 0x9b05688cu, 0x1f83d9abu, 0x5be0cd19u};
    uint8_t block[64];
    size_t fill = 0;
    uint64_t length = 0;

    static uint32_t rotr(uint32_t x, int n) { return (x >> n) | (x << (32 - n)); }

    void compress(const uint8_t* p) {
        static const uint32_t k[64] = {
            0x428a2f98u, 0x71374491u, 0xb5c0fbcfu, 0xe9b5dba5u, 0x3956c25bu, 0x59f111f1u, 0x923f82a4u,
            0xab1c5ed5u, 0xd807aa98u, 0x12835b01u, 0x243185beu, 0x550c7dc3u, 0x72be5d74u, 0x80deb1feu,
            0x9bdc06a7u, 0xc19bf174u, 0xe49b69c1u, 0xefbe4786u, 0x0fc19dc6u, 0x240ca1ccu, 0x2de92c6fu,
            0x4a7484aau, 0x5cb0a9dcu, 0x76f988dau, 0x983e5152u, 0xa831c66du, 0xb00327c8u, 0xbf597fc7u,
            0xc6e00bf3u, 0xd5a79147u, 0x06ca6351u, 0x14292967u, 0x27b70a85u, 0x2e1b2138u, 0x4d2c6dfcu,
            0x53380d13u, 0x650a7354u, 0x766a0abbu, 0x81c2c92eu, 0x92722c85u, 0xa2bfe8a1u, 0xa81a664bu,
            0xc24b8b70u, 0xc76c51a3u, 0xd192e819u, 0xd6990624u, 0xf40e3585u, 0x106aa070u, 0x19a4c116u,
            0x1e376c08u, 0x2748774cu, 0x34b0bcb5u, 0x391c0cb3u, 0x4ed8aa4au, 0x5b9cca4fu, 0x682e6ff3u,
            0x748f82eeu, 0x78a5636fu, 0x84c87814u, 0x8cc70208u, 0x90befffau, 0xa4506cebu, 0xbef9a3f7u,
            0xc67178f2u};
        uint32_t w[64];
        for (int i = 0; i < 16; ++i) {
            w[i] = (uint32_t(p[4 * i]) << 24) | (uint32_t(p[4 * i + 1]) << 16) |
                   (uint32_t(p[4 * i + 2]) << 8) | uint32_t(p[4 * i + 3]);
        }
        for (int i = 16; i < 64; ++i) {
            const uint32_t s0 = rotr(w[i - 15], 7) ^ rotr(w[i - 15], 18) ^ (w[i - 15] >> 3);
            const uint32_t s1 = rotr(w[i - 2], 17) ^ rotr(w[i - 2], 19) ^ (w[i - 2] >> 10);
            w[i] = w[i - 16] + s0 + w[i - 7] + s1;
        }
        uint32_t a = h[0], b = h[1], c = h[2], d = h[3], e = h[4], f = h[5], g = h[6], hh = h[7];
        for (int i = 0; i < 64; ++i) {
            const uint32_t s1 = rotr(e, 6) ^ rotr(e, 11) ^ rotr(e, 25);
            const uint32_t ch = (e & f) ^ (~e & g);
            const uint32_t t1 = hh + s1 + ch + k[i] + w[i];
            const uint32_t s0 = rotr(a, 2) ^ rotr(a, 13) ^ rotr(a, 22);
            const uint32_t maj = (a & b) ^ (a & c) ^ (b & c);
            const uint32_t t2 = s0 + maj;
            hh = g; g = f; f = e; e = d + t1; d = c; c = b; b = a; a = t1 + t2;
        }
        h[0] += a; h[1] += b; h[2] += c; h[3] += d; h[4] += e; h[5] += f; h[6] += g; h[7] += hh;
    }

    void update(const void* data, size_t size) {
        const uint8_t* p = static_cast<const uint8_t*>(data);
        length += size;
        if (fill > 0) {
            const size_t take = std::min(size, 64 - fill);
            std::memcpy(block + fill, p, take);
            fill += take; p += take; size -= take;
            if (fill == 64) { compress(block); fill = 0; }
        }
        while (size >= 64) { compress(p); p += 64; size -= 64; }
        if (size > 0) { std::memcpy(block, p, size); fill = size; }
    }

    std::array<uint8_t, 32> finish() {
        const uint64_t bits = length * 8;
        const uint8_t one = 0x80, zero = 0;
        update(&one, 1);
        while (fill != 56) update(&zero, 1);
        uint8_t len[8];
        for (int i = 0; i < 8; ++i) len[i] = uint8_t(bits >> (56 - 8 * i));
        update(len, 8);
        std::array<uint8_t, 32> out{};
        for (int i = 0; i < 8; ++i) {
            out[4 * i] = uint8_t(h[i] >> 24); out[4 * i + 1] = uint8_t(h[i] >> 16);
            out[4 * i + 2] = uint8_t(h[i] >> 8); out[4 * i + 3] = uint8_t(h[i]);
        }
        return out;
    }
};

// ---------------------------------------------------------------- little-endian helpers
uint32_t rd32(const uint8_t* p) { return uint32_t(p[0]) | uint32_t(p[1]) << 8 | uint32_t(p[2]) << 16 | uint32_t(p[3]) << 24; }
uint64_t rd64(const uint8_t* p) { uint64_t v = 0; for (int i = 0; i < 8; ++i) v |= uint64_t(p[i]) << (8 * i); return v; }
void put32(std::vector<uint8_t>& o, uint32_t v) { for (int i = 0; i < 4; ++i) o.push_back(uint8_t(v >> (8 * i))); }
void put64(std::vector<uint8_t>& o, uint64_t v) { for (int i = 0; i < 8; ++i) o.push_back(uint8_t(v >> (8 * i))); }
void pad(std::vector<uint8_t>& o, size_t a) { while (o.size() % a) o.push_back(0); }
bool fits(uint64_t off, uint64_t len, uint64_t size) { return off <= size && len <= size - off; }
bool all_zero(const uint8_t* p, size_t n) { for (size_t i = 0; i < n; ++i) if (p[i]) return false; return true; }

[[noreturn]] void fail(Status s, const std::string& m) { throw Error(s, m); }

struct SegmentRecord {
    uint32_t kind;
    int32_t layer;
    uint64_t tensor_count, tensor_bytes, file_size;
    std::array<uint8_t, 32> sha;
    std::string path;
};

bool safe_path(const std::string& p) {
    if (p.empty() || p.size() > 255 || p[0] == '.') return false;
    for (char c : p) if (c == '/' || c == '\\' || c == '\0') return false;
    return true;
}

bool selected(const SegmentRecord& s, uint32_t start, uint32_t end, uint32_t layers) {
    switch (s.kind) {
    case kMetadata: case kShared: return true;
    case kInput: return start == 0;
    case kLayer: return s.layer >= 0 && uint32_t(s.layer) >= start && uint32_t(s.layer) < end;
    case kOutput: return end == layers;
    default: return false;
    }
}

}  // namespace

bool type_layout(uint32_t type, uint32_t* block_elements, uint32_t* block_bytes) {
    // docs/jfm-v2-format.md:83-90 (ids 1..35).
    static const uint16_t elements[36] = {0, 1, 1, 32, 32, 32, 32, 32, 32, 256, 256, 256, 256, 256, 256, 256, 256, 256,
                                          256, 32, 256, 256, 256, 1, 1, 1, 1, 1, 256, 1, 256, 256, 32, 64, 128, 64};
    static const uint16_t bytes[36] = {0, 4, 2, 18, 20, 22, 24, 34, 36, 84, 110, 144, 176, 210, 292, 66, 74, 98,
                                       50, 18, 110, 82, 136, 1, 2, 4, 8, 8, 56, 2, 54, 66, 17, 36, 18, 18};
    if (type == 0 || type >= 36) return false;
    if (block_elements) *block_elements = elements[type];
    if (block_bytes) *block_bytes = bytes[type];
    return true;
}

const char* type_name(uint32_t type) {
    switch (type) {
    case kF32: return "F32";
    case kF16: return "F16";
    case kQ8_0: return "Q8_0";
    case kQ2_K: return "Q2_K";
    case kQ4_K: return "Q4_K";
    case kQ6_K: return "Q6_K";
    default: return "unsupported";
    }
}

std::array<uint8_t, 32> sha256(const void* data, size_t size) {
    Sha256 s;
    s.update(data, size);
    return s.finish();
}

std::string hex(const uint8_t* data, size_t size) {
    static const char* digits = "0123456789abcdef";
    std::string out;
    for (size_t i = 0; i < size; ++i) { out.push_back(digits[data[i] >> 4]); out.push_back(digits[data[i] & 15]); }
    return out;
}

// ---------------------------------------------------------------- reader
std::unique_ptr<Package> Package::open(const std::string& dir, const StagePlan& plan_in) {
    if (dir.empty()) fail(Status::InvalidArgument, "package path is required");
    const int dfd = ::open(dir.c_str(), O_RDONLY | O_DIRECTORY | O_CLOEXEC | O_NOFOLLOW);
    if (dfd < 0) fail(Status::IoError, "open package " + dir + ": " + std::strerror(errno));
    struct Closer { int fd; ~Closer() { ::close(fd); } } closer{dfd};

    auto read_file = [&](const std::string& name, size_t limit) {
        const int fd = ::openat(dfd, name.c_str(), O_RDONLY | O_CLOEXEC | O_NOFOLLOW);
        if (fd < 0) fail(Status::IoError, "open " + name + ": " + std::strerror(errno));
        struct stat st{};
        if (::fstat(fd, &st) != 0 || !S_ISREG(st.st_mode) || uint64_t(st.st_size) > limit) {
            ::close(fd);
            fail(Status::FormatError, name + " is not a bounded regular file");
        }
        std::vector<uint8_t> bytes(size_t(st.st_size));
        size_t off = 0;
        while (off < bytes.size()) {
            const ssize_t n = ::read(fd, bytes.data() + off, bytes.size() - off);
            if (n < 0 && errno == EINTR) continue;
            if (n <= 0) { ::close(fd); fail(Status::IoError, "read " + name); }
            off += size_t(n);
        }
        ::close(fd);
        return bytes;
    };

    const std::vector<uint8_t> m = read_file("manifest.jfm", kMaxManifest);
    if (m.size() < kManifestHeader || std::memcmp(m.data(), "JFMODEL2", 8) != 0 ||
        rd32(m.data() + 8) != kFormatVersion || rd32(m.data() + 60) != 0) {
        fail(Status::FormatError, "manifest has an unsupported header");
    }
    const uint32_t layers = rd32(m.data() + 12);
    const uint64_t source_size = rd64(m.data() + 16);
    const uint32_t segment_count = rd32(m.data() + 56);
    StagePlan plan = plan_in;
    if (plan.layer_end == UINT32_MAX) plan.layer_end = layers;
    if (layers == 0 || layers > kMaxLayers || source_size == 0 || plan.layer_start >= plan.layer_end ||
        plan.layer_end > layers) {
        fail(Status::InvalidArgument, "stage range or model dimensions are invalid");
    }
    if (segment_count < layers + 3 || segment_count > layers + 4) {
        fail(Status::FormatError, "manifest segment topology is invalid");
    }

    std::vector<SegmentRecord> segs;
    std::vector<uint8_t> seen(layers, 0);
    size_t cur = kManifestHeader;
    uint32_t n_meta = 0, n_shared = 0, n_in = 0, n_out = 0;
    auto pkg = std::unique_ptr<Package>(new Package());
    PackageStats& st = pkg->stats_;
    for (uint32_t i = 0; i < segment_count; ++i) {
        if (!fits(cur, kManifestRecord, m.size())) fail(Status::FormatError, "manifest segment index is truncated");
        const uint8_t* r = m.data() + cur;
        SegmentRecord s;
        s.kind = rd32(r);
        s.layer = int32_t(rd32(r + 4));
        s.tensor_count = rd64(r + 8);
        s.tensor_bytes = rd64(r + 16);
        s.file_size = rd64(r + 24);
        std::memcpy(s.sha.data(), r + 32, 32);
        const uint32_t path_len = rd32(r + 64);
        const uint32_t reserved = rd32(r + 68);
        cur += kManifestRecord;
        if (!fits(cur, path_len, m.size())) fail(Status::FormatError, "manifest contains an invalid segment");
        s.path.assign(reinterpret_cast<const char*>(m.data() + cur), path_len);
        cur += path_len;
        if (!safe_path(s.path) || s.file_size == 0 || s.kind > kMetadata || reserved != 0 ||
            (s.kind != kMetadata && (s.tensor_count == 0 || s.tensor_bytes == 0))) {
            fail(Status::FormatError, "manifest contains an invalid segment");
        }
        if (s.kind == kLayer) {
            if (s.layer < 0 || uint32_t(s.layer) >= layers || seen[size_t(s.layer)]) {
                fail(Status::FormatError, "manifest layer topology is invalid");
            }
            seen[size_t(s.layer)] = 1;
        } else {
            if (s.layer != -1) fail(Status::FormatError, "global segment declares a layer");
            if (s.kind == kShared) ++n_shared;
            if (s.kind == kInput) ++n_in;
            if (s.kind == kOutput) ++n_out;
            if (s.kind == kMetadata) {
                ++n_meta;
                if (s.tensor_count != 0 || s.tensor_bytes != 0) fail(Status::FormatError, "metadata segment declares tensors");
            }
        }
        st.total_tensor_count += s.tensor_count;
        st.total_weight_bytes += s.tensor_bytes;
        if (st.total_tensor_count > kMaxTensors) fail(Status::FormatError, "manifest tensor totals overflow");
        if (selected(s, plan.layer_start, plan.layer_end, layers)) {
            st.selected_tensor_count += s.tensor_count;
            st.selected_weight_bytes += s.tensor_bytes;
            st.mapped_bytes += s.file_size;
        }
        segs.push_back(std::move(s));
    }
    if (cur != m.size() || n_meta != 1 || n_shared > 1 || n_in != 1 || n_out != 1) {
        fail(Status::FormatError, "manifest does not define one complete model");
    }
    for (uint32_t l = 0; l < layers; ++l) {
        if (!seen[l]) fail(Status::FormatError, "manifest is missing a model layer");
    }
    {
        std::vector<std::string> paths;
        for (const auto& s : segs) paths.push_back(s.path);
        std::sort(paths.begin(), paths.end());
        if (std::adjacent_find(paths.begin(), paths.end()) != paths.end()) {
            fail(Status::FormatError, "manifest contains duplicate segment paths");
        }
    }
    std::memcpy(pkg->source_sha256_.data(), m.data() + 24, 32);
    st.layer_start = plan.layer_start;
    st.layer_end = plan.layer_end;
    st.layer_count = layers;

    for (const SegmentRecord& s : segs) {
        if (!selected(s, plan.layer_start, plan.layer_end, layers)) continue;
        const int fd = ::openat(dfd, s.path.c_str(), O_RDONLY | O_CLOEXEC | O_NOFOLLOW);
        if (fd < 0) fail(Status::IoError, "open " + s.path + ": " + std::strerror(errno));
        struct stat fst{};
        if (::fstat(fd, &fst) != 0 || !S_ISREG(fst.st_mode) || uint64_t(fst.st_size) != s.file_size) {
            ::close(fd);
            fail(Status::FormatError, s.path + " size or file type does not match manifest");
        }
        void* addr = ::mmap(nullptr, size_t(fst.st_size), PROT_READ, MAP_PRIVATE, fd, 0);
        ::close(fd);
        if (addr == MAP_FAILED) fail(Status::IoError, "map " + s.path);
        pkg->mappings_.push_back({addr, size_t(fst.st_size)});
        const uint8_t* b = static_cast<const uint8_t*>(addr);
        const uint64_t size = uint64_t(fst.st_size);
        if (plan.verify_hashes && sha256(b, size_t(size)) != s.sha) {
            fail(Status::FormatError, s.path + " checksum does not match manifest");
        }
        if (s.kind == kMetadata) {
            if (size < 4 || std::memcmp(b, "GGUF", 4) != 0) fail(Status::FormatError, "metadata segment is not a GGUF header");
            pkg->gguf_ = b;
            pkg->gguf_size_ = size_t(size);
            continue;
        }
        if (size < kSegmentHeader || std::memcmp(b, "JFSEGM02", 8) != 0 || rd32(b + 8) != kFormatVersion ||
            !all_zero(b + 32, 32)) {
            fail(Status::FormatError, "tensor segment has an unsupported header");
        }
        const uint32_t count = rd32(b + 12);
        const uint64_t index_bytes = rd64(b + 16);
        const uint64_t payload = rd64(b + 24);
        if (count != s.tensor_count || payload != s.tensor_bytes || !fits(kSegmentHeader, index_bytes, size)) {
            fail(Status::FormatError, "tensor segment has an invalid index");
        }
        const uint64_t index_end = kSegmentHeader + index_bytes;
        const uint64_t data_start = (index_end + kAlign - 1) / kAlign * kAlign;
        if (data_start > size) fail(Status::FormatError, "tensor segment data starts past end of file");
        uint64_t c = kSegmentHeader, prev_end = data_start, total = 0;
        for (uint32_t t = 0; t < count; ++t) {
            if (!fits(c, kTensorRecord, index_end)) fail(Status::FormatError, "tensor record is truncated");
            const uint8_t* r = b + c;
            TensorView v;
            v.type = rd32(r);
            v.rank = rd32(r + 4);
            v.layer = int32_t(rd32(r + 8));
            const uint32_t flags = rd32(r + 12);
            const uint64_t off = rd64(r + 48), len = rd64(r + 56);
            const uint32_t name_len = rd32(r + 64), be = rd32(r + 68), bb = rd32(r + 72), res = rd32(r + 76);
            c += kTensorRecord;
            uint32_t cbe = 0, cbb = 0;
            if (!type_layout(v.type, &cbe, &cbb) || be != cbe || bb != cbb || flags != 0 || res != 0 || v.rank == 0 ||
                v.rank > 4 || name_len == 0 || name_len > 1024 || !fits(c, name_len, index_end) || off % kAlign != 0 ||
                off < prev_end || !fits(off, len, size)) {
                fail(Status::FormatError, "tensor segment contains an invalid record");
            }
            if ((s.kind == kLayer && v.layer != s.layer) || (s.kind != kLayer && v.layer != -1)) {
                fail(Status::FormatError, "tensor layer does not match its segment");
            }
            uint64_t rows = 1;
            for (int d = 0; d < 4; ++d) {
                v.shape[d] = rd64(r + 16 + 8 * d);
                if (v.shape[d] == 0 || (uint32_t(d) >= v.rank && v.shape[d] != 1)) {
                    fail(Status::FormatError, "tensor shape is invalid");
                }
                if (d > 0) {
                    if (rows > UINT64_MAX / v.shape[d]) fail(Status::FormatError, "tensor shape overflows");
                    rows *= v.shape[d];
                }
            }
            if (v.shape[0] % be != 0) fail(Status::FormatError, "tensor storage size is inconsistent");
            const uint64_t row_bytes = v.shape[0] / be * bb;
            if (rows != 0 && row_bytes > UINT64_MAX / rows) fail(Status::FormatError, "tensor storage size is inconsistent");
            if (row_bytes * rows != len) fail(Status::FormatError, "tensor storage size is inconsistent");
            v.name.assign(reinterpret_cast<const char*>(b + c), name_len);
            v.data = b + off;
            v.size = len;
            prev_end = off + len;
            total += len;
            c = (c + name_len + 7) & ~uint64_t(7);
            pkg->tensors_.push_back(std::move(v));
        }
        if (c != index_end || total != s.tensor_bytes) {
            fail(Status::FormatError, "tensor index or payload total does not match manifest");
        }
    }
    if (pkg->tensors_.size() != st.selected_tensor_count) {
        fail(Status::FormatError, "selected tensor index is incomplete or ambiguous");
    }
    std::sort(pkg->tensors_.begin(), pkg->tensors_.end(),
              [](const TensorView& a, const TensorView& b) { return a.name < b.name; });
    for (size_t i = 1; i < pkg->tensors_.size(); ++i) {
        if (pkg->tensors_[i - 1].name == pkg->tensors_[i].name) {
            fail(Status::FormatError, "selected tensor index is incomplete or ambiguous");
        }
    }
    return pkg;
}

Package::~Package() {
    for (const Mapping& m : mappings_) ::munmap(m.address, m.size);
}

const TensorView* Package::find(const std::string& name) const {
    auto it = std::lower_bound(tensors_.begin(), tensors_.end(), name,
                               [](const TensorView& v, const std::string& n) { return v.name < n; });
    return it != tensors_.end() && it->name == name ? &*it : nullptr;
}

// ---------------------------------------------------------------- GGUF
namespace {
enum GgufType : uint32_t {
    G_U8 = 0, G_I8 = 1, G_U16 = 2, G_I16 = 3, G_U32 = 4, G_I32 = 5, G_F32 = 6, G_BOOL = 7,
    G_STR = 8, G_ARR = 9, G_U64 = 10, G_I64 = 11, G_F64 = 12,
};

size_t scalar_size(uint32_t t) {
    switch (t) {
    case G_U8: case G_I8: case G_BOOL: return 1;
    case G_U16: case G_I16: return 2;
    case G_U32: case G_I32: case G_F32: return 4;
    case G_U64: case G_I64: case G_F64: return 8;
    default: return 0;
    }
}
}  // namespace

std::map<std::string, GgufValue> parse_gguf_kv(const uint8_t* data, size_t size, bool arrays) {
    size_t c = 0;
    auto need = [&](size_t n) { if (!fits(c, n, size)) fail(Status::FormatError, "GGUF metadata is truncated"); };
    auto str = [&]() {
        need(8);
        const uint64_t n = rd64(data + c);
        c += 8;
        need(n);
        std::string s(reinterpret_cast<const char*>(data + c), size_t(n));
        c += size_t(n);
        return s;
    };
    need(24);
    if (std::memcmp(data, "GGUF", 4) != 0) fail(Status::FormatError, "metadata is not GGUF");
    const uint32_t version = rd32(data + 4);
    if (version < 2 || version > 3) fail(Status::FormatError, "unsupported GGUF version");
    c = 16;
    const uint64_t kv_count = rd64(data + c);
    c += 8;
    std::map<std::string, GgufValue> out;
    for (uint64_t i = 0; i < kv_count; ++i) {
        const std::string key = str();
        need(4);
        const uint32_t type = rd32(data + c);
        c += 4;
        GgufValue v;
        if (type == G_U32) {
            need(4); v.kind = GgufValue::U32; v.u32 = rd32(data + c); c += 4; out[key] = v;
        } else if (type == G_F32) {
            need(4); uint32_t bits = rd32(data + c); c += 4;
            v.kind = GgufValue::F32; std::memcpy(&v.f32, &bits, 4); out[key] = v;
        } else if (type == G_STR) {
            v.kind = GgufValue::Str; v.str = str(); out[key] = v;
        } else if (type == G_BOOL || type == G_I32) {
            const size_t es = scalar_size(type);
            need(es);
            v.kind = type == G_BOOL ? GgufValue::Bool : GgufValue::I32;
            v.u32 = type == G_BOOL ? data[c] : rd32(data + c);
            c += es;
            out[key] = v;
        } else if (type == G_ARR) {
            need(12);
            const uint32_t et = rd32(data + c);
            const uint64_t n = rd64(data + c + 4);
            c += 12;
            if (et == G_STR) {
                if (n > size / 8) fail(Status::FormatError, "GGUF array is invalid");
                if (arrays) {
                    v.kind = GgufValue::StrArr;
                    v.strs.reserve(size_t(n));
                    for (uint64_t k = 0; k < n; ++k) v.strs.push_back(str());
                    out[key] = std::move(v);
                } else {
                    for (uint64_t k = 0; k < n; ++k) (void) str();
                }
            } else {
                const size_t es = scalar_size(et);
                if (es == 0 || n > size / es) fail(Status::FormatError, "GGUF array is invalid");
                need(size_t(n) * es);
                if (arrays && (et == G_I32 || et == G_U32)) {
                    v.kind = GgufValue::I32Arr;
                    v.ints.resize(size_t(n));
                    for (size_t k = 0; k < size_t(n); ++k) v.ints[k] = static_cast<int32_t>(rd32(data + c + 4 * k));
                    out[key] = std::move(v);
                }
                c += size_t(n) * es;
            }
        } else {
            const size_t es = scalar_size(type);
            if (es == 0) fail(Status::FormatError, "GGUF value type is invalid");
            need(es);
            c += es;
        }
    }
    return out;
}

uint32_t jfm_type_from_ggml(uint32_t t) {
    switch (t) {
    case 0: return kF32;
    case 1: return kF16;
    case 8: return kQ8_0;
    case 10: return kQ2_K;
    case 12: return kQ4_K;
    case 14: return kQ6_K;
    default: return UINT32_MAX;
    }
}

uint32_t ggml_type_from_jfm(uint32_t t) {
    switch (t) {
    case kF32: return 0;
    case kF16: return 1;
    case kQ8_0: return 8;
    case kQ2_K: return 10;
    case kQ4_K: return 12;
    case kQ6_K: return 14;
    default: return UINT32_MAX;
    }
}

GgufLayout parse_gguf_layout(const uint8_t* data, size_t size) {
    size_t c = 0;
    auto need = [&](size_t n) { if (!fits(c, n, size)) fail(Status::FormatError, "GGUF header is truncated"); };
    auto str = [&]() {
        need(8);
        const uint64_t n = rd64(data + c);
        c += 8;
        need(n);
        std::string s(reinterpret_cast<const char*>(data + c), size_t(n));
        c += size_t(n);
        return s;
    };
    need(24);
    if (std::memcmp(data, "GGUF", 4) != 0) fail(Status::FormatError, "file is not GGUF");
    const uint32_t version = rd32(data + 4);
    if (version < 2 || version > 3) fail(Status::FormatError, "unsupported GGUF version");
    const uint64_t n_tensors = rd64(data + 8), n_kv = rd64(data + 16);
    c = 24;
    GgufLayout out;
    for (uint64_t i = 0; i < n_kv; ++i) {
        const std::string key = str();
        need(4);
        const uint32_t type = rd32(data + c);
        c += 4;
        if (type == G_STR) {
            (void) str();
        } else if (type == G_ARR) {
            need(12);
            const uint32_t et = rd32(data + c);
            const uint64_t n = rd64(data + c + 4);
            c += 12;
            if (et == G_STR) {
                for (uint64_t k = 0; k < n; ++k) (void) str();
            } else {
                const size_t es = scalar_size(et);
                if (es == 0 || n > size / es) fail(Status::FormatError, "GGUF array is invalid");
                need(size_t(n) * es);
                c += size_t(n) * es;
            }
        } else {
            const size_t es = scalar_size(type);
            if (es == 0) fail(Status::FormatError, "GGUF value type is invalid");
            need(es);
            if (key == "general.alignment") {
                if (type != G_U32) fail(Status::FormatError, "general.alignment must be u32");
                out.alignment = rd32(data + c);
                if (out.alignment == 0 || (out.alignment & (out.alignment - 1)) != 0) {
                    fail(Status::FormatError, "general.alignment must be a power of two");
                }
            }
            c += es;
        }
    }
    if (n_tensors > size / 24) fail(Status::FormatError, "GGUF tensor count is invalid");
    for (uint64_t i = 0; i < n_tensors; ++i) {
        GgufTensorInfo t;
        t.name = str();
        need(4);
        t.rank = rd32(data + c);
        c += 4;
        if (t.rank == 0 || t.rank > 4) fail(Status::FormatError, "GGUF tensor rank must be 1..4: " + t.name);
        need(8 * size_t(t.rank) + 12);
        for (uint32_t d = 0; d < t.rank; ++d) t.shape[d] = rd64(data + c + 8 * d);
        c += 8 * size_t(t.rank);
        t.type = rd32(data + c);
        t.offset = rd64(data + c + 4);
        c += 12;
        out.tensors.push_back(std::move(t));
    }
    out.data_offset = (uint64_t(c) + out.alignment - 1) / out.alignment * out.alignment;
    return out;
}

std::shared_ptr<const MappedFile> MappedFile::open(const std::string& path) {
    const int fd = ::open(path.c_str(), O_RDONLY | O_CLOEXEC);
    if (fd < 0) fail(Status::IoError, "open " + path + ": " + std::strerror(errno));
    struct stat st{};
    if (::fstat(fd, &st) != 0 || !S_ISREG(st.st_mode) || st.st_size <= 0) {
        ::close(fd);
        fail(Status::IoError, path + " is not a regular, non-empty file");
    }
    void* addr = ::mmap(nullptr, size_t(st.st_size), PROT_READ, MAP_PRIVATE, fd, 0);
    ::close(fd);
    if (addr == MAP_FAILED) fail(Status::IoError, "map " + path);
    auto m = std::shared_ptr<MappedFile>(new MappedFile());
    m->data_ = static_cast<const uint8_t*>(addr);
    m->size_ = size_t(st.st_size);
    return m;
}

MappedFile::~MappedFile() {
    if (data_) ::munmap(const_cast<uint8_t*>(data_), size_);
}

std::vector<uint8_t> write_gguf_header(const std::vector<std::pair<std::string, GgufValue>>& kv,
                                       const std::vector<GgufTensorInfo>& tensors) {
    std::vector<uint8_t> o;
    o.insert(o.end(), {'G', 'G', 'U', 'F'});
    put32(o, 3);
    put64(o, tensors.size());
    put64(o, kv.size());
    auto put_str = [&](const std::string& s) { put64(o, s.size()); o.insert(o.end(), s.begin(), s.end()); };
    for (const auto& [key, v] : kv) {
        put_str(key);
        switch (v.kind) {
        case GgufValue::U32: put32(o, G_U32); put32(o, v.u32); break;
        case GgufValue::F32: { put32(o, G_F32); uint32_t bits; std::memcpy(&bits, &v.f32, 4); put32(o, bits); break; }
        case GgufValue::Str: put32(o, G_STR); put_str(v.str); break;
        case GgufValue::Bool: put32(o, G_BOOL); o.push_back(v.u32 ? 1 : 0); break;
        case GgufValue::I32: put32(o, G_I32); put32(o, v.u32); break;
        case GgufValue::StrArr:
            put32(o, G_ARR); put32(o, G_STR); put64(o, v.strs.size());
            for (const std::string& e : v.strs) put_str(e);
            break;
        case GgufValue::I32Arr:
            put32(o, G_ARR); put32(o, G_I32); put64(o, v.ints.size());
            for (const int32_t e : v.ints) put32(o, static_cast<uint32_t>(e));
            break;
        }
    }
    for (const GgufTensorInfo& t : tensors) {
        put_str(t.name);
        put32(o, t.rank);
        for (uint32_t d = 0; d < t.rank; ++d) put64(o, t.shape[d]);
        const uint32_t ggml = ggml_type_from_jfm(t.type);
        if (ggml == UINT32_MAX) fail(Status::InvalidArgument, "tensor type has no GGML id: " + t.name);
        put32(o, ggml);
        put64(o, t.offset);
    }
    pad(o, 32);
    return o;
}

// ---------------------------------------------------------------- writer
std::pair<std::array<uint8_t, 32>, uint64_t> source_digest(const std::vector<uint8_t>& gguf_header,
                                                           const std::vector<TensorBlob>& tensors) {
    Sha256 src;
    src.update(gguf_header.data(), gguf_header.size());
    uint64_t size = gguf_header.size();
    static const uint8_t zeros[32] = {};
    uint64_t data_pos = 0;
    for (const TensorBlob& t : tensors) {
        while (data_pos % 32) {
            src.update(zeros, 1);
            ++data_pos;
            ++size;
        }
        src.update(t.data, size_t(t.size));
        data_pos += t.size;
        size += t.size;
    }
    return {src.finish(), size};
}

void write_package(const std::string& dir, uint32_t layer_count, const std::vector<uint8_t>& gguf_header,
                   const std::vector<TensorBlob>& tensors,
                   const std::pair<std::array<uint8_t, 32>, uint64_t>* source) {
    namespace fs = std::filesystem;
    std::error_code ec;
    fs::create_directories(dir, ec);
    if (ec) fail(Status::IoError, "create package directory " + dir + ": " + ec.message());

    struct Group {
        uint32_t kind;
        int32_t layer;
        std::string path;
        std::vector<const TensorBlob*> members;
    };
    std::map<std::string, Group> groups;
    for (const TensorBlob& t : tensors) {
        Group g{kShared, -1, "shared.jfs", {}};
        if (t.name.rfind("blk.", 0) == 0) {
            const size_t dot = t.name.find('.', 4);
            const int32_t layer = std::stoi(t.name.substr(4, dot - 4));
            char path[32];
            std::snprintf(path, sizeof(path), "layer-%05d.jfs", layer);
            g = Group{kLayer, layer, path, {}};
        } else if (t.name.rfind("token_embd.", 0) == 0) {
            g = Group{kInput, -1, "input.jfs", {}};
        } else if (t.name.rfind("output.", 0) == 0 || t.name.rfind("output_norm.", 0) == 0) {
            g = Group{kOutput, -1, "output.jfs", {}};
        }
        auto [it, inserted] = groups.emplace(g.path, g);
        it->second.members.push_back(&t);
    }

    struct Written {
        uint32_t kind;
        int32_t layer;
        uint64_t count, bytes, size;
        std::array<uint8_t, 32> sha;
        std::string path;
    };
    std::vector<Written> written;
    auto write_file = [&](const std::string& name, const std::vector<uint8_t>& head,
                          const std::vector<std::pair<const uint8_t*, uint64_t>>& payloads, uint64_t total_size) {
        std::ofstream f(fs::path(dir) / name, std::ios::binary | std::ios::trunc);
        if (!f) fail(Status::IoError, "create " + name);
        Sha256 h;
        f.write(reinterpret_cast<const char*>(head.data()), std::streamsize(head.size()));
        h.update(head.data(), head.size());
        uint64_t pos = head.size();
        static const uint8_t zeros[64] = {};
        for (const auto& [p, n] : payloads) {
            while (pos % kAlign) { f.write(reinterpret_cast<const char*>(zeros), 1); h.update(zeros, 1); ++pos; }
            f.write(reinterpret_cast<const char*>(p), std::streamsize(n));
            h.update(p, size_t(n));
            pos += n;
        }
        while (pos < total_size) { f.write(reinterpret_cast<const char*>(zeros), 1); h.update(zeros, 1); ++pos; }
        if (!f) fail(Status::IoError, "write " + name);
        return h.finish();
    };

    {  // metadata.gguf
        Written w{kMetadata, -1, 0, 0, gguf_header.size(), {}, "metadata.gguf"};
        w.sha = write_file(w.path, gguf_header, {}, gguf_header.size());
        written.push_back(w);
    }
    auto emit = [&](Group& g) {
        std::sort(g.members.begin(), g.members.end(),
                  [](const TensorBlob* a, const TensorBlob* b) { return a->name < b->name; });
        std::vector<uint8_t> index;
        for (const TensorBlob* t : g.members) {
            index.resize(index.size() + kTensorRecord, 0);
            index.insert(index.end(), t->name.begin(), t->name.end());
            pad(index, 8);
        }
        const uint64_t data_start = (kSegmentHeader + index.size() + kAlign - 1) / kAlign * kAlign;
        std::vector<uint8_t> head;
        head.insert(head.end(), {'J', 'F', 'S', 'E', 'G', 'M', '0', '2'});
        put32(head, kFormatVersion);
        put32(head, uint32_t(g.members.size()));
        put64(head, index.size());
        uint64_t payload_total = 0;
        for (const TensorBlob* t : g.members) payload_total += t->size;
        put64(head, payload_total);
        head.resize(kSegmentHeader, 0);
        // fill records now that offsets are known
        uint64_t off = data_start, c = 0;
        std::vector<std::pair<const uint8_t*, uint64_t>> payloads;
        for (const TensorBlob* t : g.members) {
            std::vector<uint8_t> r;
            uint32_t be = 0, bb = 0;
            type_layout(t->type, &be, &bb);
            put32(r, t->type);
            put32(r, t->rank);
            put32(r, uint32_t(g.layer));
            put32(r, 0);
            for (int d = 0; d < 4; ++d) put64(r, t->shape[d]);
            put64(r, off);
            put64(r, t->size);
            put32(r, uint32_t(t->name.size()));
            put32(r, be);
            put32(r, bb);
            put32(r, 0);
            std::memcpy(index.data() + c, r.data(), kTensorRecord);
            c = (c + kTensorRecord + t->name.size() + 7) & ~uint64_t(7);
            payloads.emplace_back(t->data, t->size);
            off = (off + t->size + kAlign - 1) / kAlign * kAlign;
        }
        head.insert(head.end(), index.begin(), index.end());
        const uint64_t file_size = off;
        Written w{g.kind, g.layer, g.members.size(), payload_total, file_size, {}, g.path};
        w.sha = write_file(g.path, head, payloads, file_size);
        written.push_back(w);
    };
    auto take = [&](const std::string& path) {
        auto it = groups.find(path);
        if (it == groups.end()) fail(Status::InvalidArgument, "package is missing tensors for " + path);
        emit(it->second);
        groups.erase(it);
    };
    take("input.jfs");
    for (uint32_t l = 0; l < layer_count; ++l) {
        char path[32];
        std::snprintf(path, sizeof(path), "layer-%05u.jfs", l);
        take(path);
    }
    take("output.jfs");
    if (groups.count("shared.jfs")) take("shared.jfs");
    if (!groups.empty()) fail(Status::InvalidArgument, "tensor belongs to a layer outside the model");

    const auto [src_sha, src_size] = source ? *source : source_digest(gguf_header, tensors);

    std::vector<uint8_t> man;
    man.insert(man.end(), {'J', 'F', 'M', 'O', 'D', 'E', 'L', '2'});
    put32(man, kFormatVersion);
    put32(man, layer_count);
    put64(man, src_size);
    man.insert(man.end(), src_sha.begin(), src_sha.end());
    put32(man, uint32_t(written.size()));
    put32(man, 0);
    for (const Written& w : written) {
        put32(man, w.kind);
        put32(man, uint32_t(w.layer));
        put64(man, w.count);
        put64(man, w.bytes);
        put64(man, w.size);
        man.insert(man.end(), w.sha.begin(), w.sha.end());
        put32(man, uint32_t(w.path.size()));
        put32(man, 0);
        man.insert(man.end(), w.path.begin(), w.path.end());
    }
    std::ofstream f(fs::path(dir) / "manifest.jfm", std::ios::binary | std::ios::trunc);
    f.write(reinterpret_cast<const char*>(man.data()), std::streamsize(man.size()));
    if (!f) fail(Status::IoError, "write manifest.jfm");
}

}  // namespace jfh
