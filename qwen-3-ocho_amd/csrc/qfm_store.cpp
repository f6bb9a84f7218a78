// qfm_store.cpp -- the mmap'd weight store: the reference's manifest index or
// safetensors files read directly.
//
// Everything is validated once at open, so that a lookup can hand out
// shard_maps[file_idx] + data_off without further checks: each entry lies
// inside its mapped shard, names are unique and NUL-terminated, and each
// safetensors entry's byte count matches its shape and dtype. Lookups are a
// binary search over the entries sorted by strcmp, as the reference's
// (ocho/amd_server/reader.cpp:63-72).
#include "qfm_internal.h"
#include "../../include/qf_store.h"

#include <dirent.h>
#include <fcntl.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <algorithm>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <string>
#include <vector>

static_assert(sizeof(QfRec) == 88, "QfRec layout");
static_assert(sizeof(QfEntry) == QF_REC_SIZE, "QfEntry must be a 512-byte record");
static_assert(offsetof(QfEntry, rec) == QF_MAX_NAME, "QfEntry layout");
static_assert(offsetof(QfRec, data_off) == 40 && offsetof(QfRec, scale2_file) == 72, "QfRec layout");
static_assert(sizeof(QfRouteMailbox) == 136, "QfRouteMailbox layout");

using namespace qfm;

namespace {

// ---- a minimal JSON reader for safetensors headers ---------------------------
// Only what a header holds: one object whose members are objects with
// "dtype" (string), "shape" (array of integers) and "data_offsets" (two
// integers); "__metadata__" and unknown members are skipped.
struct Json {
    const char *p, *end;
    bool ok = true;

    void ws() {
        while (p < end && (*p == ' ' || *p == '\t' || *p == '\n' || *p == '\r')) p++;
    }
    bool eat(char c) {
        ws();
        if (p < end && *p == c) { p++; return true; }
        return false;
    }
    bool str(std::string &out) {
        ws();
        out.clear();
        if (p >= end || *p != '"') return ok = false;
        p++;
        while (p < end && *p != '"') {
            char c = *p++;
            if (c != '\\') { out.push_back(c); continue; }
            if (p >= end) return ok = false;
            const char e = *p++;
            switch (e) {
                case '"': out.push_back('"'); break;
                case '\\': out.push_back('\\'); break;
                case '/': out.push_back('/'); break;
                case 'b': out.push_back('\b'); break;
                case 'f': out.push_back('\f'); break;
                case 'n': out.push_back('\n'); break;
                case 'r': out.push_back('\r'); break;
                case 't': out.push_back('\t'); break;
                case 'u': {
                    if (end - p < 4) return ok = false;
                    unsigned v = 0;
                    for (int i = 0; i < 4; i++) {
                        const char h = *p++;
                        v <<= 4;
                        if (h >= '0' && h <= '9') v |= (unsigned)(h - '0');
                        else if (h >= 'a' && h <= 'f') v |= (unsigned)(h - 'a' + 10);
                        else if (h >= 'A' && h <= 'F') v |= (unsigned)(h - 'A' + 10);
                        else return ok = false;
                    }
                    // names are ASCII in practice; other code points are kept as UTF-8
                    if (v < 0x80) out.push_back((char)v);
                    else if (v < 0x800) { out.push_back((char)(0xC0 | (v >> 6))); out.push_back((char)(0x80 | (v & 63))); }
                    else {
                        out.push_back((char)(0xE0 | (v >> 12)));
                        out.push_back((char)(0x80 | ((v >> 6) & 63)));
                        out.push_back((char)(0x80 | (v & 63)));
                    }
                    break;
                }
                default: return ok = false;
            }
        }
        if (p >= end) return ok = false;
        p++;
        return true;
    }
    // non-negative integer below 2^63
    bool uint(uint64_t &v) {
        ws();
        if (p >= end || *p < '0' || *p > '9') return ok = false;
        v = 0;
        while (p < end && *p >= '0' && *p <= '9') {
            const uint64_t d = (uint64_t)(*p++ - '0');
            if (v > (((uint64_t)1 << 63) - 1 - d) / 10) return ok = false;
            v = v * 10 + d;
        }
        if (p < end && (*p == '.' || *p == 'e' || *p == 'E')) return ok = false;
        return true;
    }
    bool skip(int depth = 0) {
        ws();
        if (p >= end || depth > 64) return ok = false;
        const char c = *p;
        if (c == '"') { std::string s; return str(s); }
        if (c == '{' || c == '[') {
            const char close = c == '{' ? '}' : ']';
            p++;
            if (eat(close)) return true;
            do {
                if (c == '{') {
                    std::string k;
                    if (!str(k) || !eat(':')) return ok = false;
                }
                if (!skip(depth + 1)) return false;
            } while (eat(','));
            return eat(close) ? true : (ok = false);
        }
        // number / true / false / null
        const char *q = p;
        while (p < end && (std::strchr("+-.eE0123456789", *p) || (*p >= 'a' && *p <= 'z'))) p++;
        return p > q ? true : (ok = false);
    }
};

struct DtInfo { const char *name; uint32_t code; uint32_t size; };
const DtInfo kDtypes[] = {
    {"BF16", QF_DT_BF16, 2}, {"F32", QF_DT_F32, 4}, {"U8", QF_DT_U8, 1}, {"F8_E4M3", QF_DT_F8_E4M3, 1},
    {"I64", QF_DT_I64, 8}, {"F16", QF_DT_F16, 2}, {"I8", QF_DT_I8, 1}, {"I32", QF_DT_I32, 4},
    {"F64", QF_DT_F64, 8}, {"F8_E5M2", QF_DT_F8_E5M2, 1}, {"I16", QF_DT_I16, 2}, {"U16", QF_DT_U16, 2},
    {"U32", QF_DT_U32, 4}, {"U64", QF_DT_U64, 8}, {"BOOL", QF_DT_BOOL, 1},
};

int fail(int code, const char *fmt, const char *a, const char *b = "") {
    set_error(code, fmt, a, b);
    return code;
}

// Parse one safetensors file (mapped at base, size bytes) into entries.
int parse_safetensors(const char *path, const uint8_t *base, size_t size, uint32_t shard,
                      std::vector<QfEntry> &out) {
    if (size < 8) return fail(-5, "qf_store_open: %s: shorter than a safetensors header%s", path);
    uint64_t n = 0;
    for (int i = 7; i >= 0; i--) n = (n << 8) | base[i];
    if (n < 2 || n > size - 8 || n > ((uint64_t)100 << 20))
        return fail(-5, "qf_store_open: %s: header length out of range%s", path);
    const uint64_t data0 = 8 + n, data_bytes = size - data0;
    Json j{reinterpret_cast<const char *>(base + 8), reinterpret_cast<const char *>(base + 8 + n)};
    if (!j.eat('{')) return fail(-5, "qf_store_open: %s: header is not a JSON object%s", path);
    if (j.eat('}')) return 0;
    do {
        std::string name;
        if (!j.str(name) || !j.eat(':')) return fail(-5, "qf_store_open: %s: malformed header%s", path);
        if (name == "__metadata__") {
            if (!j.skip()) return fail(-5, "qf_store_open: %s: malformed __metadata__%s", path);
            continue;
        }
        if (name.empty() || name.size() >= QF_MAX_NAME)
            return fail(-5, "qf_store_open: %s: tensor name empty or longer than 255 bytes: %s", path, name.c_str());
        if (!j.eat('{')) return fail(-5, "qf_store_open: %s: entry %s is not an object", path, name.c_str());
        std::string dtype;
        std::vector<uint64_t> shape, offs;
        bool have_dt = false, have_shape = false, have_offs = false;
        if (!j.eat('}')) {
            do {
                std::string key;
                if (!j.str(key) || !j.eat(':')) return fail(-5, "qf_store_open: %s: malformed entry %s", path, name.c_str());
                if (key == "dtype") {
                    if (!j.str(dtype)) return fail(-5, "qf_store_open: %s: bad dtype of %s", path, name.c_str());
                    have_dt = true;
                } else if (key == "shape" || key == "data_offsets") {
                    std::vector<uint64_t> &v = key == "shape" ? shape : offs;
                    if (!j.eat('[')) return fail(-5, "qf_store_open: %s: bad array in %s", path, name.c_str());
                    if (!j.eat(']')) {
                        do {
                            uint64_t x;
                            if (!j.uint(x) || v.size() > 8) return fail(-5, "qf_store_open: %s: bad integer in %s", path, name.c_str());
                            v.push_back(x);
                        } while (j.eat(','));
                        if (!j.eat(']')) return fail(-5, "qf_store_open: %s: bad array in %s", path, name.c_str());
                    }
                    (key == "shape" ? have_shape : have_offs) = true;
                } else if (!j.skip()) {
                    return fail(-5, "qf_store_open: %s: malformed entry %s", path, name.c_str());
                }
            } while (j.eat(','));
            if (!j.eat('}')) return fail(-5, "qf_store_open: %s: malformed entry %s", path, name.c_str());
        }
        if (!have_dt || !have_shape || !have_offs || offs.size() != 2)
            return fail(-5, "qf_store_open: %s: entry %s lacks dtype, shape or data_offsets", path, name.c_str());
        const DtInfo *dt = nullptr;
        for (const DtInfo &d : kDtypes)
            if (dtype == d.name) dt = &d;
        if (!dt) return fail(-5, "qf_store_open: %s: unsupported dtype of %s", path, name.c_str());
        if (shape.size() > 4) return fail(-5, "qf_store_open: %s: %s has more than 4 dimensions", path, name.c_str());
        uint64_t count = 1;
        for (uint64_t d : shape) {
            if (d && count > (UINT64_MAX / 16) / d) return fail(-5, "qf_store_open: %s: shape of %s overflows", path, name.c_str());
            count *= d;
        }
        if (offs[1] < offs[0] || offs[1] > data_bytes)
            return fail(-5, "qf_store_open: %s: data_offsets of %s outside the file", path, name.c_str());
        if (offs[1] - offs[0] != count * dt->size)
            return fail(-5, "qf_store_open: %s: byte count of %s does not match its shape and dtype", path, name.c_str());
        QfEntry e;
        std::memset(&e, 0, sizeof e);
        std::memcpy(e.name, name.data(), name.size());
        e.rec.file_idx = shard;
        e.rec.dtype = dt->code;
        for (int d = 0; d < 4; d++) e.rec.ne[d] = 1;
        for (size_t d = 0; d < shape.size(); d++) e.rec.ne[d] = shape[shape.size() - 1 - d];   // fastest first
        e.rec.data_off = data0 + offs[0];
        e.rec.nbytes = offs[1] - offs[0];
        out.push_back(e);
    } while (j.eat(','));
    if (!j.eat('}') || !j.ok) return fail(-5, "qf_store_open: %s: malformed header%s", path);
    return 0;
}

bool ends_with(const std::string &s, const char *suf) {
    const size_t n = std::strlen(suf);
    return s.size() >= n && s.compare(s.size() - n, n, suf) == 0;
}

bool is_dir(const char *p) {
    struct stat sb {};
    return stat(p, &sb) == 0 && S_ISDIR(sb.st_mode);
}
bool is_file(const char *p) {
    struct stat sb {};
    return stat(p, &sb) == 0 && S_ISREG(sb.st_mode);
}

int map_shards(QfStore *st, const std::vector<std::string> &paths) {
    const int n = (int)paths.size();
    st->n_shards = n;
    st->shard_paths = (char(*)[1024])std::calloc(n ? n : 1, 1024);
    st->shard_fds = (int *)std::malloc((size_t)(n ? n : 1) * sizeof(int));
    st->shard_maps = (void **)std::calloc(n ? n : 1, sizeof(void *));
    st->shard_sizes = (size_t *)std::calloc(n ? n : 1, sizeof(size_t));
    if (!st->shard_paths || !st->shard_fds || !st->shard_maps || !st->shard_sizes) return fail(-4, "qf_store_open: out of host memory%s%s", "");
    for (int i = 0; i < n; i++) st->shard_fds[i] = -1;
    for (int i = 0; i < n; i++) {
        if (paths[i].size() >= 1024) return fail(-3, "qf_store_open: shard path too long: %s%s", paths[i].c_str());
        std::memcpy(st->shard_paths[i], paths[i].c_str(), paths[i].size() + 1);
        st->shard_fds[i] = open(paths[i].c_str(), O_RDONLY);
        if (st->shard_fds[i] < 0) return fail(-3, "qf_store_open: cannot open shard %s%s", paths[i].c_str());
        struct stat sb {};
        if (fstat(st->shard_fds[i], &sb) != 0) return fail(-3, "qf_store_open: cannot stat shard %s%s", paths[i].c_str());
        st->shard_sizes[i] = (size_t)sb.st_size;
        if (st->shard_sizes[i] == 0) continue;   // nothing can point into an empty shard
        void *m = mmap(nullptr, st->shard_sizes[i], PROT_READ, MAP_PRIVATE, st->shard_fds[i], 0);
        if (m == MAP_FAILED) return fail(-4, "qf_store_open: cannot map shard %s%s", paths[i].c_str());
        st->shard_maps[i] = m;
    }
    return 0;
}

const QfEntry *find_in(const QfEntry *v, int n, const char *name) {
    int lo = 0, hi = n - 1;
    while (lo <= hi) {
        const int mid = lo + (hi - lo) / 2;
        const int c = std::strcmp(v[mid].name, name);
        if (c == 0) return &v[mid];
        if (c < 0) lo = mid + 1;
        else hi = mid - 1;
    }
    return nullptr;
}

int open_manifest(QfStore *st, const std::string &dir) {
    std::vector<std::string> paths;
    FILE *f = std::fopen((dir + "/shards.txt").c_str(), "r");
    if (!f) return fail(-1, "qf_store_open: %s/shards.txt not found%s", dir.c_str());
    char line[1100];
    while (std::fgets(line, sizeof line, f)) {
        line[std::strcspn(line, "\r\n")] = 0;
        if (line[0]) paths.emplace_back(line);
    }
    std::fclose(f);
    f = std::fopen((dir + "/manifest.bin").c_str(), "rb");
    if (!f) return fail(-2, "qf_store_open: %s/manifest.bin not readable%s", dir.c_str());
    std::fseek(f, 0, SEEK_END);
    const long sz = std::ftell(f);
    std::fseek(f, 0, SEEK_SET);
    if (sz < 0 || sz % QF_REC_SIZE) {
        std::fclose(f);
        return fail(-2, "qf_store_open: %s/manifest.bin is not a whole number of 512-byte records%s", dir.c_str());
    }
    st->n_entries = (int)(sz / QF_REC_SIZE);
    st->entries = (QfEntry *)std::malloc(sz ? (size_t)sz : 1);
    if (!st->entries || (sz && std::fread(st->entries, 1, (size_t)sz, f) != (size_t)sz)) {
        std::fclose(f);
        return fail(-2, "qf_store_open: %s/manifest.bin read failed%s", dir.c_str());
    }
    std::fclose(f);
    const int rc = map_shards(st, paths);
    if (rc) return rc;
    for (int i = 0; i < st->n_entries; i++) {
        const QfEntry &e = st->entries[i];
        if (!std::memchr(e.name, 0, QF_MAX_NAME)) return fail(-5, "qf_store_open: manifest record %s has no NUL in its name%s", std::to_string(i).c_str());
        const QfRec &r = e.rec;
        if (r.file_idx >= (uint32_t)st->n_shards || r.data_off > st->shard_sizes[r.file_idx] ||
            r.nbytes > st->shard_sizes[r.file_idx] - r.data_off)
            return fail(-5, "qf_store_open: manifest entry %s lies outside its shard%s", e.name);
        if ((r.scale2_off && (r.scale2_file >= (uint32_t)st->n_shards || r.scale2_off > st->shard_sizes[r.scale2_file] ||
                              st->shard_sizes[r.scale2_file] - r.scale2_off < 4)) ||
            (r.input_off && (r.input_file >= (uint32_t)st->n_shards || r.input_off > st->shard_sizes[r.input_file] ||
                             st->shard_sizes[r.input_file] - r.input_off < 4)))
            return fail(-5, "qf_store_open: manifest entry %s has a scale offset outside its shard%s", e.name);
    }
    std::sort(st->entries, st->entries + st->n_entries,
              [](const QfEntry &a, const QfEntry &b) { return std::strcmp(a.name, b.name) < 0; });
    for (int i = 1; i < st->n_entries; i++)
        if (!std::strcmp(st->entries[i - 1].name, st->entries[i].name))
            return fail(-5, "qf_store_open: duplicate tensor %s%s", st->entries[i].name);
    return 0;
}

int open_safetensors(QfStore *st, const std::string &path) {
    std::vector<std::string> paths;
    if (is_dir(path.c_str())) {
        DIR *d = opendir(path.c_str());
        if (!d) return fail(-1, "qf_store_open: cannot list %s%s", path.c_str());
        while (dirent *de = readdir(d)) {
            const std::string nm = de->d_name;
            const std::string full = path + "/" + nm;
            if (ends_with(nm, ".safetensors") && is_file(full.c_str())) paths.push_back(full);
        }
        closedir(d);
        std::sort(paths.begin(), paths.end());
        if (paths.empty()) return fail(-1, "qf_store_open: %s holds neither shards.txt nor .safetensors files%s", path.c_str());
    } else if (is_file(path.c_str())) {
        paths.push_back(path);
    } else {
        return fail(-1, "qf_store_open: %s does not exist%s", path.c_str());
    }
    int rc = map_shards(st, paths);
    if (rc) return rc;
    std::vector<QfEntry> ents;
    for (int i = 0; i < st->n_shards; i++) {
        rc = parse_safetensors(st->shard_paths[i], (const uint8_t *)st->shard_maps[i], st->shard_sizes[i], (uint32_t)i, ents);
        if (rc) return rc;
    }
    std::sort(ents.begin(), ents.end(), [](const QfEntry &a, const QfEntry &b) { return std::strcmp(a.name, b.name) < 0; });
    for (size_t i = 1; i < ents.size(); i++)
        if (!std::strcmp(ents[i - 1].name, ents[i].name)) return fail(-5, "qf_store_open: duplicate tensor %s%s", ents[i].name);
    // companion scales of NVFP4 weights: X.weight -> X.weight_scale_2 / X.input_scale (4-byte F32)
    for (QfEntry &e : ents) {
        if (!ends_with(e.name, ".weight")) continue;
        const std::string stem(e.name, std::strlen(e.name) - 7);
        const QfEntry *s2 = find_in(ents.data(), (int)ents.size(), (stem + ".weight_scale_2").c_str());
        const QfEntry *in = find_in(ents.data(), (int)ents.size(), (stem + ".input_scale").c_str());
        if (s2 && s2->rec.dtype == QF_DT_F32 && s2->rec.nbytes == 4) {
            e.rec.scale2_off = s2->rec.data_off;
            e.rec.scale2_file = s2->rec.file_idx;
        }
        if (in && in->rec.dtype == QF_DT_F32 && in->rec.nbytes == 4) {
            e.rec.input_off = in->rec.data_off;
            e.rec.input_file = in->rec.file_idx;
        }
    }
    st->n_entries = (int)ents.size();
    st->entries = (QfEntry *)std::malloc(ents.size() ? ents.size() * sizeof(QfEntry) : 1);
    if (!st->entries) return fail(-4, "qf_store_open: out of host memory%s%s", "");
    if (!ents.empty()) std::memcpy(st->entries, ents.data(), ents.size() * sizeof(QfEntry));
    return 0;
}

}  // namespace

extern "C" {

void qf_store_close(QfStore *st) {
    if (!st) return;
    for (int i = 0; i < st->n_shards; i++) {
        if (st->shard_maps && st->shard_maps[i] && st->shard_maps[i] != MAP_FAILED)
            munmap(st->shard_maps[i], st->shard_sizes[i]);
        if (st->shard_fds && st->shard_fds[i] >= 0) close(st->shard_fds[i]);
    }
    std::free(st->shard_paths);
    std::free(st->shard_fds);
    std::free(st->shard_maps);
    std::free(st->shard_sizes);
    std::free(st->entries);
    std::memset(st, 0, sizeof *st);
}

int qf_store_open(QfStore *st, const char *path) {
    if (!st || !path) { set_error(-1, "qf_store_open: null argument"); return -1; }
    std::memset(st, 0, sizeof *st);
    std::string p(path);
    while (p.size() > 1 && p.back() == '/') p.pop_back();
    const bool manifest = is_dir(p.c_str()) && is_file((p + "/shards.txt").c_str());
    const int rc = manifest ? open_manifest(st, p) : open_safetensors(st, p);
    if (rc) qf_store_close(st);
    return rc;
}

const QfEntry *qf_find(const QfStore *st, const char *name) {
    if (!st || !name || !st->entries) return nullptr;
    return find_in(st->entries, st->n_entries, name);
}

const void *qfm_store_data(const QfStore *st, const QfEntry *e) {
    if (!st || !e || e->rec.file_idx >= (uint32_t)st->n_shards || !st->shard_maps[e->rec.file_idx]) return nullptr;
    return (const uint8_t *)st->shard_maps[e->rec.file_idx] + e->rec.data_off;
}

}  // extern "C"
