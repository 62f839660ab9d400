// .cmf v2 container reader (host side): the fixed envelope, the binary tensor
// directory, zero-copy tensor bytes over a read-only mapping of the file,
// integrity hashes and shard merging.  Follows cortiq-core/src/format.rs
// (CmfModel::open :390-584, parse_envelope :653-728, decode_directory
// :730-798, tensor_index :809-821, entry_bytes :924-933, verify :1063-1110,
// open_sharded :589-650) and hash.rs (hash64).  Every validation failure is an
// error with the kind of the reference's CmfError; nothing is defaulted.
//
// The header JSON is checked for well-formed JSON syntax here; its fields
// (arch, shard coordinates, section hashes) are read by the host binding,
// which hands the stored section hashes back to cmf_file_verify.
#include <fcntl.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <algorithm>
#include <cctype>
#include <cerrno>
#include <cinttypes>
#include <cstdio>
#include <cstring>
#include <string>
#include <unordered_map>
#include <vector>

#include "../../include/cmf_hip.h"
#include "common.h"

namespace cmf {
namespace {

constexpr uint8_t kMagic[4] = {'C', 'M', 'F', 0x01};
constexpr uint32_t kVersion = 2;
constexpr size_t kEnvelopeLen = 128, kRecordLen = 56, kMaxNdim = 6;
constexpr uint64_t kDataAlign = 4096, kTensorAlign = 64;
// required_features this reader implements: TENSOR_DIR | BINARY_MASKS |
// QUANT_2F | LOOP_MASKS | SKILL_FILE (format.rs:54-75)
constexpr uint32_t kSupported = (1u << 0) | (1u << 1) | (1u << 2) | (1u << 5) | (1u << 6);
constexpr int kGroup = 32;

uint64_t fmix64(uint64_t x) {
    x ^= x >> 33;
    x *= 0xFF51AFD7ED558CCDull;
    x ^= x >> 33;
    x *= 0xC4CEB9FE1A85EC53ull;
    x ^= x >> 33;
    return x;
}

uint64_t le64(const uint8_t* p) {
    uint64_t v;
    std::memcpy(&v, p, 8);
    return v;
}
uint32_t le32(const uint8_t* p) {
    uint32_t v;
    std::memcpy(&v, p, 4);
    return v;
}
uint16_t le16(const uint8_t* p) {
    uint16_t v;
    std::memcpy(&v, p, 2);
    return v;
}

int err(int code, const std::string& msg) {
    set_error(msg);
    return code;
}

std::string hex16(uint64_t v) {
    char b[17];
    std::snprintf(b, sizeof b, "%016" PRIx64, v);
    return b;
}

// Strict UTF-8 (no overlongs, no surrogates, at most U+10FFFF).
bool utf8_ok(const uint8_t* s, size_t n) {
    size_t i = 0;
    while (i < n) {
        const uint8_t c = s[i];
        if (c < 0x80) {
            i++;
            continue;
        }
        int len;
        uint32_t cp;
        if ((c & 0xE0) == 0xC0) len = 2, cp = c & 0x1F;
        else if ((c & 0xF0) == 0xE0) len = 3, cp = c & 0x0F;
        else if ((c & 0xF8) == 0xF0) len = 4, cp = c & 0x07;
        else return false;
        if (i + len > n) return false;
        for (int k = 1; k < len; k++) {
            if ((s[i + k] & 0xC0) != 0x80) return false;
            cp = (cp << 6) | (s[i + k] & 0x3F);
        }
        if ((len == 2 && cp < 0x80) || (len == 3 && cp < 0x800) || (len == 4 && cp < 0x10000)) return false;
        if (cp > 0x10FFFF || (cp >= 0xD800 && cp <= 0xDFFF)) return false;
        i += len;
    }
    return true;
}

// RFC 8259 syntax check of the header JSON (recursive descent, depth-bounded).
struct JsonCheck {
    const uint8_t* p;
    const uint8_t* e;
    int depth = 0;
    void ws() {
        while (p < e && (*p == ' ' || *p == '\t' || *p == '\n' || *p == '\r')) p++;
    }
    bool lit(const char* s) {
        const size_t n = std::strlen(s);
        if ((size_t)(e - p) < n || std::memcmp(p, s, n) != 0) return false;
        p += n;
        return true;
    }
    bool str() {
        if (p >= e || *p != '"') return false;
        p++;
        const uint8_t* s0 = p;
        while (p < e && *p != '"') {
            if (*p < 0x20) return false;
            if (*p == '\\') {
                if (++p >= e) return false;
                if (*p == 'u') {
                    for (int k = 0; k < 4; k++)
                        if (++p >= e || !std::isxdigit(*p)) return false;
                } else if (!std::strchr("\"\\/bfnrt", *p)) {
                    return false;
                }
            }
            p++;
        }
        if (p >= e || !utf8_ok(s0, p - s0)) return false;
        p++;
        return true;
    }
    bool num() {
        if (p < e && *p == '-') p++;
        if (p >= e) return false;
        if (*p == '0') p++;
        else if (*p >= '1' && *p <= '9') while (p < e && std::isdigit(*p)) p++;
        else return false;
        if (p < e && *p == '.') {
            p++;
            if (p >= e || !std::isdigit(*p)) return false;
            while (p < e && std::isdigit(*p)) p++;
        }
        if (p < e && (*p == 'e' || *p == 'E')) {
            p++;
            if (p < e && (*p == '+' || *p == '-')) p++;
            if (p >= e || !std::isdigit(*p)) return false;
            while (p < e && std::isdigit(*p)) p++;
        }
        return true;
    }
    bool value() {
        ws();
        if (p >= e) return false;
        if (*p == '{' || *p == '[') {
            if (++depth > 128) return false;
            const uint8_t close = *p == '{' ? '}' : ']';
            const bool obj = *p == '{';
            p++;
            ws();
            if (p < e && *p == close) {
                p++;
                depth--;
                return true;
            }
            for (;;) {
                if (obj) {
                    ws();
                    if (!str()) return false;
                    ws();
                    if (p >= e || *p != ':') return false;
                    p++;
                }
                if (!value()) return false;
                ws();
                if (p < e && *p == ',') {
                    p++;
                    continue;
                }
                if (p < e && *p == close) {
                    p++;
                    depth--;
                    return true;
                }
                return false;
            }
        }
        if (*p == '"') return str();
        if (*p == 't') return lit("true");
        if (*p == 'f') return lit("false");
        if (*p == 'n') return lit("null");
        return num();
    }
    bool document() {
        ws();
        if (p >= e || *p != '{') return false;  // the header is an object
        if (!value()) return false;
        ws();
        return p == e;
    }
};

// Payload length a dtype fixes for a shape (quant.rs:552-612); false where the
// reader does not define it (variable-length or reserved dtypes) or the size
// overflows.
bool expected_nbytes(int dtype, const uint64_t* shape, int ndim, uint64_t& out) {
    uint64_t n = 1;
    for (int d = 0; d < ndim; d++)
        if (__builtin_mul_overflow(n, shape[d], &n)) return false;
    auto mul = [](uint64_t a, uint64_t b, uint64_t& r) { return !__builtin_mul_overflow(a, b, &r); };
    auto add = [](uint64_t a, uint64_t b, uint64_t& r) { return !__builtin_add_overflow(a, b, &r); };
    const uint64_t groups = n / kGroup + (n % kGroup ? 1 : 0);
    uint64_t a, b;
    switch (dtype) {
        case 0: return mul(n, 4, out);                                    // f32
        case 1: case 2: return mul(n, 2, out);                            // f16, bf16
        case 3: return ndim >= 1 && mul(shape[0], 2, a) && add(n, a, out); // q8_row
        case 4: case 11: return mul(groups, 18, out);                     // q4_block, q4_tiled
        case 12: return mul(groups, 6, out);                              // q1
        case 15: case 16: {                                               // q4tp, q2tp
            if (ndim != 2 || shape[1] % kGroup) return false;
            const uint64_t rows = shape[0], gpr = shape[1] / kGroup;
            const uint64_t chunk = dtype == 15 ? 16 : 8;
            uint64_t c, st;
            if (!mul(gpr, 5, st)) return false;
            st = st / 8 + (st % 8 ? 1 : 0);
            return mul(rows, gpr, a) && mul(a, chunk, a) && mul(rows, 4, b) && add(a, b, a) && mul(rows, st, c) &&
                   add(a, c, out);
        }
        case 9: {                                                         // q8_2f
            if (ndim < 1) return false;
            const uint64_t o = shape[0], inn = n / (o ? o : 1);
            uint64_t c;
            return mul(o, 2, a) && add(n, a, a) && mul(inn, 2, c) && add(a, c, out);
        }
        default: return false;
    }
}

bool known_dtype(int id) { return id >= 0 && id <= 16; }  // TensorDtype::from_id (types.rs:101-122)

}  // namespace

uint64_t hash64_bytes(const uint8_t* b, size_t n) {
    const size_t full = n / 8;
    uint64_t acc = 0;
    for (size_t i = 0; i < full; i++) acc ^= fmix64(le64(b + 8 * i)) ^ ((uint64_t)i * 0x9E3779B97F4A7C15ull);
    const size_t rem = n % 8;
    if (rem) {
        uint8_t w[8] = {0};
        std::memcpy(w, b + 8 * full, rem);
        acc ^= fmix64(le64(w)) ^ ((uint64_t)full * 0x9E3779B97F4A7C15ull);
    }
    acc ^= (uint64_t)n;
    return fmix64(acc);
}

struct Backing {
    const uint8_t* base = nullptr;
    uint64_t len = 0;
    bool mapped = false;
    std::vector<uint8_t> owned;
    ~Backing() {
        if (mapped && base) munmap((void*)base, len);
    }
};

struct FileEntry {
    std::string name;
    int dtype, ndim;
    uint64_t shape[kMaxNdim];
    uint64_t off, nbytes, hash;
    int shard;  // 0: this file, i > 0: the i-th attached shard
};


}  // namespace cmf

struct CmfFileS {
    std::string path;
    cmf::Backing* mem = nullptr;                 // primary mapping
    std::vector<std::pair<cmf::Backing*, uint64_t>> shards;  // attached shards: mapping, data_off
    uint32_t features = 0;
    uint64_t sec[6][2] = {};  // header, dir, data, masks, vocab, index
    uint64_t header_hash = 0, dir_hash = 0;
    std::vector<cmf::FileEntry> ents;
    std::unordered_map<uint64_t, uint32_t> by_name;
    std::vector<uint32_t> overflow;
    ~CmfFileS() {
        delete mem;
        for (auto& s : shards) delete s.first;
    }
    const uint8_t* entry_data(const cmf::FileEntry& t) const {
        if (t.shard == 0) return mem->base + sec[2][0] + t.off;
        const auto& s = shards[t.shard - 1];
        return s.first->base + s.second + t.off;
    }
    int index(const char* name, size_t n) const {
        const uint64_t h = cmf::hash64_bytes((const uint8_t*)name, n);
        auto it = by_name.find(h);
        auto same = [&](uint32_t i) { return ents[i].name.size() == n && !std::memcmp(ents[i].name.data(), name, n); };
        if (it != by_name.end() && same(it->second)) return (int)it->second;
        for (uint32_t i : overflow)
            if (same(i)) return (int)i;
        return -1;
    }
    // adds entry i to the name index; false on a duplicate name
    bool index_add(uint32_t i) {
        const auto& nm = ents[i].name;
        const uint64_t h = cmf::hash64_bytes((const uint8_t*)nm.data(), nm.size());
        auto it = by_name.find(h);
        if (it == by_name.end()) {
            by_name.emplace(h, i);
            return true;
        }
        if (ents[it->second].name == nm) return false;
        for (uint32_t j : overflow)
            if (ents[j].name == nm) return false;
        overflow.push_back(i);  // distinct names with one hash
        return true;
    }
};

namespace cmf {
namespace {

int map_file(const char* path, Backing& b) {
    struct stat st;
    if (::stat(path, &st) != 0) {
        if (errno == ENOENT) return err(CMF_E_NOTFOUND, std::string("file not found: ") + path);
        return err(CMF_E_IO, std::string("stat ") + path + ": " + std::strerror(errno));
    }
    const int fd = ::open(path, O_RDONLY | O_CLOEXEC);
    if (fd < 0) return err(CMF_E_IO, std::string("open ") + path + ": " + std::strerror(errno));
    b.len = (uint64_t)st.st_size;
    if (b.len > 0) {
        void* p = ::mmap(nullptr, b.len, PROT_READ, MAP_PRIVATE, fd, 0);
        if (p != MAP_FAILED) {
            b.base = (const uint8_t*)p;
            b.mapped = true;
        } else {  // no mapping: read the file into memory
            b.owned.resize(b.len);
            size_t got = 0;
            while (got < b.len) {
                const ssize_t r = ::pread(fd, b.owned.data() + got, b.len - got, (off_t)got);
                if (r <= 0) {
                    ::close(fd);
                    return err(CMF_E_IO, std::string("read ") + path + ": " + std::strerror(errno));
                }
                got += (size_t)r;
            }
            b.base = b.owned.data();
        }
    }
    ::close(fd);
    return CMF_OK;
}

// parse_envelope (format.rs:653-728)
int parse_envelope(CmfFileS& f) {
    const uint8_t* b = f.mem->base;
    const uint64_t n = f.mem->len;
    if (n < kEnvelopeLen)
        return err(CMF_E_BOUNDS, "file too small for CMF envelope: " + std::to_string(n) + " bytes");
    if (std::memcmp(b, kMagic, 4) != 0) return err(CMF_E_MAGIC, "invalid magic (not a CMF file)");
    const uint32_t version = le32(b + 4);
    if (version != kVersion) return err(CMF_E_VERSION, "unsupported version " + std::to_string(version));
    f.features = le32(b + 12);
    const uint32_t unknown = f.features & ~kSupported;
    if (unknown) return err(CMF_E_FEATURE, "unsupported required feature bits " + std::to_string(unknown));
    static const char* names[6] = {"header", "dir", "data", "masks", "vocab", "index"};
    for (int s = 0; s < 6; s++) {
        f.sec[s][0] = le64(b + 0x10 + 16 * s);
        f.sec[s][1] = le64(b + 0x18 + 16 * s);
    }
    f.header_hash = le64(b + 0x70);
    f.dir_hash = le64(b + 0x78);
    for (int s = 0; s < 6; s++) {
        const uint64_t off = f.sec[s][0], len = f.sec[s][1];
        if (s < 2 && len == 0) return err(CMF_E_BOUNDS, std::string("section '") + names[s] + "' is required");
        uint64_t end;
        if (len > 0 && (__builtin_add_overflow(off, len, &end) || end > n))
            return err(CMF_E_BOUNDS, std::string("section '") + names[s] + "' [" + std::to_string(off) + ", " +
                                         std::to_string(off + len) + ") exceeds file (" + std::to_string(n) +
                                         " bytes)");
    }
    if (f.sec[2][1] > 0 && f.sec[2][0] % kDataAlign)
        return err(CMF_E_BOUNDS, "data section offset " + std::to_string(f.sec[2][0]) + " not 4096-aligned");
    return CMF_OK;
}

// decode_directory (format.rs:730-798)
int decode_directory(CmfFileS& f) {
    const uint8_t* d = f.mem->base + f.sec[1][0];
    const uint64_t n = f.sec[1][1];
    if (n < 16) return err(CMF_E_PARSE, "tensor directory too short");
    const uint64_t count = le64(d), pool_off = le64(d + 8);
    uint64_t rec_len, rec_end;
    if (__builtin_mul_overflow(count, (uint64_t)kRecordLen, &rec_len))
        return err(CMF_E_PARSE, "tensor directory record count overflows");
    if (__builtin_add_overflow((uint64_t)16, rec_len, &rec_end))
        return err(CMF_E_PARSE, "tensor directory size overflows");
    if (rec_end > n || pool_off > n || pool_off < rec_end)
        return err(CMF_E_PARSE, "tensor directory malformed: count=" + std::to_string(count) +
                                    ", pool_off=" + std::to_string(pool_off) + ", len=" + std::to_string(n));
    const uint8_t* pool = d + pool_off;
    const uint64_t pool_len = n - pool_off;
    f.ents.reserve(count);
    for (uint64_t i = 0; i < count; i++) {
        const uint8_t* r = d + 16 + i * kRecordLen;
        const uint64_t name_off = le32(r), name_len = le16(r + 4);
        FileEntry t{};
        t.dtype = r[6];
        t.ndim = r[7];
        if (t.ndim > (int)kMaxNdim)
            return err(CMF_E_PARSE, "tensor #" + std::to_string(i) + ": ndim " + std::to_string(t.ndim) + " > 6");
        for (int k = 0; k < t.ndim; k++) t.shape[k] = le32(r + 8 + 4 * k);
        t.off = le64(r + 32);
        t.nbytes = le64(r + 40);
        t.hash = le64(r + 48);
        if (name_off + name_len > pool_len)
            return err(CMF_E_PARSE, "tensor #" + std::to_string(i) + ": name out of pool");
        if (!utf8_ok(pool + name_off, name_len))
            return err(CMF_E_PARSE, "tensor #" + std::to_string(i) + ": name is not UTF-8");
        t.name.assign((const char*)pool + name_off, name_len);
        if (!known_dtype(t.dtype)) return err(CMF_E_DTYPE, "unknown dtype id " + std::to_string(t.dtype));
        f.ents.push_back(std::move(t));
    }
    return CMF_OK;
}

// the per-tensor checks of CmfModel::open (format.rs:460-531)
int check_tensors(CmfFileS& f) {
    for (const auto& t : f.ents) {
        const std::string q = "tensor '" + t.name + "': ";
        if (t.off % kTensorAlign) return err(CMF_E_BOUNDS, q + "offset " + std::to_string(t.off) + " not 64-aligned");
        uint64_t end;
        if (__builtin_add_overflow(t.off, t.nbytes, &end)) return err(CMF_E_BOUNDS, q + "offset + length overflows");
        if (end > f.sec[2][1])
            return err(CMF_E_BOUNDS, q + "[" + std::to_string(t.off) + ", " + std::to_string(end) +
                                         ") exceeds data section (" + std::to_string(f.sec[2][1]) + " bytes)");
        uint64_t prod = 1;
        for (int k = 0; k < t.ndim; k++)
            if (__builtin_mul_overflow(prod, t.shape[k], &prod)) return err(CMF_E_BOUNDS, q + "shape product overflows");
        uint64_t expect;
        if (expected_nbytes(t.dtype, t.shape, t.ndim, expect) && expect != t.nbytes)
            return err(CMF_E_BOUNDS, q + "nbytes " + std::to_string(t.nbytes) + " != expected " +
                                         std::to_string(expect) + " for dtype " + std::to_string(t.dtype));
    }
    for (uint32_t i = 0; i < f.ents.size(); i++)
        if (!f.index_add(i)) return err(CMF_E_PARSE, "duplicate tensor name '" + f.ents[i].name + "' in directory");
    return CMF_OK;
}

}  // namespace
}  // namespace cmf

using namespace cmf;

extern "C" {

uint64_t cmf_hash64(const void* data, size_t n) { return hash64_bytes((const uint8_t*)data, n); }

int cmf_file_open(const char* path, cmf_file* out) {
    if (!path || !out) return fail("file_open: null argument");
    *out = nullptr;
    auto* f = new CmfFileS();
    f->path = path;
    f->mem = new Backing();
    int rc = map_file(path, *f->mem);
    if (rc == CMF_OK) rc = parse_envelope(*f);
    if (rc == CMF_OK) {
        JsonCheck j{f->mem->base + f->sec[0][0], f->mem->base + f->sec[0][0] + f->sec[0][1]};
        if (!j.document()) rc = err(CMF_E_PARSE, "header JSON: malformed");
    }
    if (rc == CMF_OK) rc = decode_directory(*f);
    if (rc == CMF_OK) rc = check_tensors(*f);
    if (rc != CMF_OK) {
        delete f;
        return rc;
    }
    *out = f;
    return CMF_OK;
}

int cmf_file_close(cmf_file f) {
    delete f;
    return CMF_OK;
}

int cmf_file_info(cmf_file f, cmf_file_sections* s) {
    if (!f || !s) return fail("file_info: null argument");
    s->required_features = f->features;
    for (int k = 0; k < 6; k++) {
        s->off[k] = f->sec[k][0];
        s->len[k] = f->sec[k][1];
    }
    s->header_hash = f->header_hash;
    s->dir_hash = f->dir_hash;
    s->base = f->mem->base;
    s->file_len = f->mem->len;
    return CMF_OK;
}

int cmf_file_count(cmf_file f) { return f ? (int)f->ents.size() : fail("file_count: null file"); }

int cmf_file_entry(cmf_file f, int i, cmf_file_tensor* e) {
    if (!f || !e) return fail("file_entry: null argument");
    if (i < 0 || i >= (int)f->ents.size()) return err(CMF_E_MISSING, "file_entry: index out of range");
    const FileEntry& t = f->ents[i];
    e->name = t.name.data();
    e->name_len = (int)t.name.size();
    e->dtype = t.dtype;
    e->ndim = t.ndim;
    for (int k = 0; k < 6; k++) e->shape[k] = k < t.ndim ? t.shape[k] : 0;
    e->off = t.off;
    e->nbytes = t.nbytes;
    e->hash = t.hash;
    e->shard = t.shard;
    e->data = f->entry_data(t);
    return CMF_OK;
}

int cmf_file_find(cmf_file f, const char* name, size_t name_len) {
    if (!f || !name) return fail("file_find: null argument");
    const int i = f->index(name, name_len);
    return i >= 0 ? i : err(CMF_E_MISSING, "tensor '" + std::string(name, name_len) + "' not found in CMF directory");
}

int cmf_file_attach_shard(cmf_file f, cmf_file shard) {
    if (!f || !shard || f == shard) return fail("file_attach_shard: two distinct open files");
    const int idx = (int)f->shards.size() + 1;
    const size_t first_new = f->ents.size();
    for (const auto& t0 : shard->ents) {
        FileEntry t = t0;
        t.shard = idx;
        f->ents.push_back(std::move(t));
        if (!f->index_add((uint32_t)(f->ents.size() - 1))) {
            const std::string nm = f->ents.back().name;
            // undo: the file keeps its directory as before the call
            for (size_t i = first_new; i + 1 < f->ents.size(); i++) {
                const auto& n2 = f->ents[i].name;
                auto it = f->by_name.find(hash64_bytes((const uint8_t*)n2.data(), n2.size()));
                if (it != f->by_name.end() && it->second == i) f->by_name.erase(it);
            }
            f->overflow.erase(std::remove_if(f->overflow.begin(), f->overflow.end(),
                                             [&](uint32_t i) { return i >= first_new; }),
                              f->overflow.end());
            f->ents.resize(first_new);
            return err(CMF_E_PARSE, "duplicate tensor name '" + nm + "' across shards");
        }
    }
    f->shards.push_back({shard->mem, shard->sec[2][0]});
    shard->mem = nullptr;  // the mapping now belongs to f
    shard->ents.clear();
    delete shard;
    return CMF_OK;
}

int cmf_file_verify(cmf_file f, const uint64_t* stored, char* buf, size_t cap, int* nproblems) {
    if (!f || !nproblems) return fail("file_verify: null argument");
    std::vector<std::string> probs;
    const uint8_t* b = f->mem->base;
    auto check = [&](const char* name, uint64_t want, int s) {
        if (want != 0 && f->sec[s][1] > 0) {
            const uint64_t got = hash64_bytes(b + f->sec[s][0], f->sec[s][1]);
            if (got != want)
                probs.push_back(std::string("section '") + name + "': hash mismatch (stored " + hex16(want) +
                                ", actual " + hex16(got) + ")");
        }
    };
    check("header", f->header_hash, 0);
    check("dir", f->dir_hash, 1);
    if (stored) {
        check("masks", stored[0], 3);
        check("vocab", stored[1], 4);
        check("index", stored[2], 5);
    }
    for (const auto& t : f->ents) {
        const uint64_t got = hash64_bytes(f->entry_data(t), t.nbytes);
        if (got != t.hash)
            probs.push_back("tensor '" + t.name + "': hash mismatch (stored " + hex16(t.hash) + ", actual " +
                            hex16(got) + ")");
    }
    *nproblems = (int)probs.size();
    if (buf && cap) {
        std::string all;
        for (size_t i = 0; i < probs.size(); i++) all += (i ? "\n" : "") + probs[i];
        const size_t n = std::min(cap - 1, all.size());
        std::memcpy(buf, all.data(), n);
        buf[n] = 0;
    }
    return CMF_OK;
}

}  // extern "C"
