// gguf.cpp — GGUF reader/writer and the in-process image registry.
#include "gguf.h"
#include <fcntl.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>
#include <climits>
#include <cstring>
#include <mutex>

namespace cj {

namespace {
std::mutex g_img_mu;
std::map<std::string, std::pair<std::unique_ptr<uint8_t[]>, size_t>> g_images;

struct Rd {
    const uint8_t *p;
    size_t n, at = 0;
    bool ok = true;
    template <class T> T get() {
        T v{};
        if (at + sizeof(T) > n) { ok = false; return v; }
        memcpy(&v, p + at, sizeof(T));
        at += sizeof(T);
        return v;
    }
    std::string str() {
        uint64_t len = get<uint64_t>();
        if (!ok || len > n - at) { ok = false; return {}; }   // written so a huge len cannot wrap
        std::string s((const char *)p + at, (size_t)len);
        at += (size_t)len;
        return s;
    }
};

bool read_value(Rd &r, int type, GgufValue &v, int depth = 0) {
    v.type = type;
    switch (type) {
    case 0: v.i = r.get<uint8_t>(); break;
    case 1: v.i = r.get<int8_t>(); break;
    case 2: v.i = r.get<uint16_t>(); break;
    case 3: v.i = r.get<int16_t>(); break;
    case 4: v.i = r.get<uint32_t>(); break;
    case 5: v.i = r.get<int32_t>(); break;
    case 6: v.f = r.get<float>(); v.i = (int64_t)v.f; break;
    case 7: v.i = r.get<uint8_t>(); break;
    case 8: v.s = r.str(); break;
    case 10: v.i = (int64_t)r.get<uint64_t>(); break;
    case 11: v.i = r.get<int64_t>(); break;
    case 12: v.f = r.get<double>(); v.i = (int64_t)v.f; break;
    case 9: {
        int et = (int)r.get<uint32_t>();
        uint64_t cnt = r.get<uint64_t>();
        if (depth >= 4) return false;   // nested arrays: bounded, so a crafted header cannot exhaust the stack
        for (uint64_t k = 0; k < cnt && r.ok; k++) {
            GgufValue e;
            if (!read_value(r, et, e, depth + 1)) return false;
            if (et == 6 || et == 12) v.af.push_back(e.f);
            else if (et != 8) v.ai.push_back(e.i);
        }
    } break;
    default: return false;
    }
    if (type == 6 || type == 12) {} else if (type != 8 && type != 9) v.f = (double)v.i;
    return r.ok;
}
}  // namespace

int ggml_block_elems(int t) {
    switch (t) { case 0: case 1: return 1; case 2: case 8: case 39: return 32; case 12: case 14: return 256; default: return -1; }
}
int ggml_block_bytes(int t) {
    switch (t) { case 0: return 4; case 1: return 2; case 2: return 18; case 8: return 34; case 12: return 144; case 14: return 210; case 39: return 17; default: return -1; }
}
int64_t ggml_row_bytes(int type, int64_t cols) {
    int be = ggml_block_elems(type), bb = ggml_block_bytes(type);
    if (be < 0 || cols % be) return -1;
    return cols / be * bb;
}

Gguf::~Gguf() {
    for (auto &m : maps_) munmap(m.first, m.second);
}

namespace {
// The shard number and count a split name carries ("-00002-of-00004.gguf":
// 2 of 4, numbered from 1), or 0 when the name is not a shard's.
int split_in_name(const std::string &p, int *count) {
    const size_t tail = 20;   // "-00001-of-00004.gguf"
    if (p.size() < tail) return 0;
    const std::string t = p.substr(p.size() - tail);
    if (t[0] != '-' || t.compare(6, 4, "-of-") != 0 || t.compare(15, 5, ".gguf") != 0) return 0;
    for (int i : {1, 2, 3, 4, 5, 10, 11, 12, 13, 14})
        if (t[i] < '0' || t[i] > '9') return 0;
    *count = std::stoi(t.substr(10, 5));
    return std::stoi(t.substr(1, 5));
}

std::string shard_path(const std::string &prefix, int no, int count) {
    char tail[32];
    snprintf(tail, sizeof tail, "-%05d-of-%05d.gguf", no, count);
    return prefix + tail;
}
}  // namespace

bool Gguf::map_file(const std::string &path, const uint8_t **p, size_t *n, std::string &err) {
    int fd = ::open(path.c_str(), O_RDONLY);
    if (fd < 0) { err = "cannot open " + path; return false; }
    struct stat st;
    if (fstat(fd, &st) != 0 || st.st_size < 24) { ::close(fd); err = "cannot stat " + path; return false; }
    void *m = mmap(nullptr, (size_t)st.st_size, PROT_READ, MAP_PRIVATE, fd, 0);
    ::close(fd);
    if (m == MAP_FAILED) { err = "mmap failed for " + path; return false; }
    maps_.push_back({m, (size_t)st.st_size});
    *p = (const uint8_t *)m;
    *n = (size_t)st.st_size;
    return true;
}

bool Gguf::open(const std::string &path, std::string &err) {
    if (path.rfind("mem:", 0) == 0) {
        const uint8_t *p; size_t n;
        if (!image_get(path.substr(4), &p, &n)) { err = "no in-process image " + path; return false; }
        return parse(p, n, kv_, err);
    }
    // a later shard's name leads to shard 1, which carries the metadata
    int named = 0;
    const int no = split_in_name(path, &named);
    const std::string prefix = no > 0 ? path.substr(0, path.size() - 20) : path;
    const std::string root = no > 1 ? shard_path(prefix, 1, named) : path;
    const uint8_t *p; size_t n;
    if (!map_file(root, &p, &n, err)) {
        if (no > 1) err = "gguf: '" + path + "' is shard " + std::to_string(no) + " of " + std::to_string(named) +
                          " and shard 1, which carries the model metadata, is missing - expected '" + root + "'";
        return false;
    }
    if (!parse(p, n, kv_, err)) return false;
    const int64_t count = get_int("split.count", 1);
    if (count <= 1) return true;
    if (get_int("split.no", 0) != 0) { err = "gguf: '" + root + "' carries the model metadata but is not split 0"; return false; }
    if (no == 0 || named != count) {
        err = "gguf: '" + root + "' declares split.count " + std::to_string(count) +
              " but its name does not follow <base>-%05d-of-%05d.gguf for that count";
        return false;
    }
    for (int k = 2; k <= (int)count; k++) {
        const std::string sp = shard_path(prefix, k, (int)count);
        std::string e2;
        if (!map_file(sp, &p, &n, e2)) {
            int have = 1;
            for (int j = 2; j <= (int)count; j++) if (::access(shard_path(prefix, j, (int)count).c_str(), R_OK) == 0) have++;
            err = "gguf: shard " + std::to_string(k) + " of " + std::to_string(count) + " is missing - expected '" + sp +
                  "'; found " + std::to_string(have) + " of " + std::to_string(count) +
                  " shards. Refusing to load a truncated model.";
            return false;
        }
        std::map<std::string, GgufValue> skv;
        if (!parse(p, n, skv, err)) return false;
        auto it = skv.find("split.no");
        if (it == skv.end() || it->second.i != k - 1) {
            err = "gguf: '" + sp + "' does not declare split.no " + std::to_string(k - 1);
            return false;
        }
    }
    const int64_t want = get_int("split.tensors.count", (int64_t)tensors_.size());
    if (want != (int64_t)tensors_.size()) {
        err = "gguf: the shards hold " + std::to_string(tensors_.size()) + " tensors, split.tensors.count says " +
              std::to_string(want);
        return false;
    }
    return true;
}

bool Gguf::parse(const uint8_t *p, size_t n, std::map<std::string, GgufValue> &kv, std::string &err) {
    Rd r{p, n};
    if (r.get<uint32_t>() != 0x46554747u) { err = "not a GGUF file (magic)"; return false; }
    uint32_t ver = r.get<uint32_t>();
    if (ver != 2 && ver != 3) { err = "GGUF version " + std::to_string(ver) + " is not 2 or 3"; return false; }
    uint64_t nt = r.get<uint64_t>(), nkv = r.get<uint64_t>();
    for (uint64_t i = 0; i < nkv && r.ok; i++) {
        std::string k = r.str();
        int ty = (int)r.get<uint32_t>();
        GgufValue v;
        if (!read_value(r, ty, v)) { err = "bad metadata value for " + k; return false; }
        kv[k] = std::move(v);
    }
    const size_t first = tensors_.size();
    for (uint64_t i = 0; i < nt && r.ok; i++) {
        GgufTensor t;
        t.name = r.str();
        uint32_t nd = r.get<uint32_t>();
        if (nd > 4) { err = "tensor " + t.name + " has " + std::to_string(nd) + " dims"; return false; }
        int64_t elems = 1;
        for (uint32_t d = 0; d < nd; d++) {
            const uint64_t v = r.get<uint64_t>();
            // every extent positive, and the element count representable
            if (r.ok && (v == 0 || v > (uint64_t)INT64_MAX / (uint64_t)elems)) {
                err = "tensor " + t.name + ": dimension " + std::to_string(d) + " is " + std::to_string(v) +
                      (v == 0 ? "" : ", which overflows the element count");
                return false;
            }
            elems *= (int64_t)v;
            t.dims.push_back((int64_t)v);
        }
        t.type = (int)r.get<uint32_t>();
        t.offset = r.get<uint64_t>();
        tensors_.push_back(std::move(t));
    }
    if (!r.ok) { err = "truncated GGUF header"; return false; }
    // alignment: io/GgufFile.cajeta:773-777 (each file's own)
    auto al = kv.find("general.alignment");
    uint64_t align = al != kv.end() ? (uint64_t)al->second.i : 32;
    if (align == 0) align = 32;
    if (align > (1u << 20)) { err = "general.alignment " + std::to_string(align) + " is not served (at most 1 MiB)"; return false; }
    uint64_t data = (r.at + align - 1) / align * align;
    if (data > n) { err = "truncated GGUF: no tensor data"; return false; }
    for (size_t i = first; i < tensors_.size(); i++) {
        GgufTensor &t = tensors_[i];
        int64_t rb = ggml_row_bytes(t.type, t.cols());
        if (rb < 0) { err = "tensor " + t.name + ": type " + std::to_string(t.type) + " is not served"; return false; }
        if (t.dims.empty() || t.rows() > INT64_MAX / rb) { err = "tensor " + t.name + ": byte size overflows"; return false; }
        t.bytes = rb * t.rows();
        // written so that no sum can wrap: data <= n is checked above
        if (t.offset > n - data || (uint64_t)t.bytes > n - data - t.offset) {
            err = "tensor " + t.name + " runs past the end of the file";
            return false;
        }
        t.data = p + data + t.offset;
        if (index_.count(t.name)) { err = "tensor " + t.name + " appears twice"; return false; }
        index_[t.name] = i;
    }
    return true;
}

const GgufTensor *Gguf::tensor(const std::string &name) const {
    auto it = index_.find(name);
    return it == index_.end() ? nullptr : &tensors_[it->second];
}
const GgufValue *Gguf::get(const std::string &key) const {
    auto it = kv_.find(key);
    return it == kv_.end() ? nullptr : &it->second;
}
int64_t Gguf::get_int(const std::string &key, int64_t dflt) const {
    const GgufValue *v = get(key);
    return v ? v->i : dflt;
}
double Gguf::get_float(const std::string &key, double dflt) const {
    const GgufValue *v = get(key);
    return v ? v->f : dflt;
}
std::string Gguf::get_str(const std::string &key, const std::string &dflt) const {
    const GgufValue *v = get(key);
    return v && v->type == 8 ? v->s : dflt;
}

// ---------------------------------------------------------------- writer

namespace {
void put_bytes(std::vector<uint8_t> &o, const void *p, size_t n) {
    const uint8_t *b = (const uint8_t *)p;
    o.insert(o.end(), b, b + n);
}
template <class T> void put(std::vector<uint8_t> &o, T v) { put_bytes(o, &v, sizeof v); }
void put_str(std::vector<uint8_t> &o, const std::string &s) {
    put<uint64_t>(o, s.size());
    put_bytes(o, s.data(), s.size());
}
}  // namespace

void GgufWriter::kv_u32(const std::string &k, uint32_t v) { put_str(meta_, k); put<uint32_t>(meta_, 4); put(meta_, v); n_kv_++; }
void GgufWriter::kv_i32(const std::string &k, int32_t v) { put_str(meta_, k); put<uint32_t>(meta_, 5); put(meta_, v); n_kv_++; }
void GgufWriter::kv_f32(const std::string &k, float v) { put_str(meta_, k); put<uint32_t>(meta_, 6); put(meta_, v); n_kv_++; }
void GgufWriter::kv_bool(const std::string &k, bool v) { put_str(meta_, k); put<uint32_t>(meta_, 7); put<uint8_t>(meta_, v ? 1 : 0); n_kv_++; }
void GgufWriter::kv_str(const std::string &k, const std::string &v) { put_str(meta_, k); put<uint32_t>(meta_, 8); put_str(meta_, v); n_kv_++; }

void GgufWriter::tensor(const std::string &name, int type, std::vector<int64_t> dims) {
    T t{name, type, std::move(dims), 0, 0};
    int64_t rows = 1;
    for (size_t i = 1; i < t.dims.size(); i++) rows *= t.dims[i];
    t.bytes = ggml_row_bytes(type, t.dims[0]) * rows;
    ts_.push_back(std::move(t));
}

size_t GgufWriter::layout(std::vector<size_t> &offsets) {
    size_t hdr = 4 + 4 + 8 + 8 + meta_.size();
    for (auto &t : ts_) hdr += 8 + t.name.size() + 4 + 8 * t.dims.size() + 4 + 8;
    const size_t align = 32;
    header_size_ = (hdr + align - 1) / align * align;
    uint64_t off = 0;
    offsets.clear();
    for (auto &t : ts_) {
        t.off = off;
        offsets.push_back(header_size_ + off);
        off += ((uint64_t)t.bytes + align - 1) / align * align;
    }
    return header_size_ + off;
}

void GgufWriter::write_header(uint8_t *out) const {
    std::vector<uint8_t> h;
    put<uint32_t>(h, 0x46554747u);
    put<uint32_t>(h, 3);
    put<uint64_t>(h, ts_.size());
    put<uint64_t>(h, n_kv_);
    put_bytes(h, meta_.data(), meta_.size());
    for (auto &t : ts_) {
        put_str(h, t.name);
        put<uint32_t>(h, (uint32_t)t.dims.size());
        for (int64_t d : t.dims) put<uint64_t>(h, (uint64_t)d);
        put<uint32_t>(h, (uint32_t)t.type);
        put<uint64_t>(h, t.off);
    }
    h.resize(header_size_, 0);
    memcpy(out, h.data(), h.size());
}

// ---------------------------------------------------------------- images

uint8_t *image_create(const std::string &name, size_t bytes) {
    std::unique_ptr<uint8_t[]> p(new (std::nothrow) uint8_t[bytes]);
    if (!p) return nullptr;
    uint8_t *raw = p.get();
    std::lock_guard<std::mutex> lk(g_img_mu);
    g_images[name] = {std::move(p), bytes};
    return raw;
}
bool image_get(const std::string &name, const uint8_t **p, size_t *n) {
    std::lock_guard<std::mutex> lk(g_img_mu);
    auto it = g_images.find(name);
    if (it == g_images.end()) return false;
    *p = it->second.first.get();
    *n = it->second.second;
    return true;
}
bool image_free(const std::string &name) {
    std::lock_guard<std::mutex> lk(g_img_mu);
    return g_images.erase(name) != 0;
}

}  // namespace cj
