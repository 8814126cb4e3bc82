// gguf.h — a minimal GGUF v2/v3 reader (file mmap or in-process image) and
// writer, enough for LlmEngine.load's llama-architecture keys
// (model/ModelConfig.cajeta:172-320) and the tensor table
// (io/GgufFile.cajeta, alignment :773-777).
#pragma once
#include <cstdint>
#include <map>
#include <memory>
#include <string>
#include <vector>

namespace cj {

struct GgufTensor {
    std::string name;
    int type = 0;
    std::vector<int64_t> dims;   // ne[0] (columns) first
    uint64_t offset = 0;         // from the data section
    int64_t bytes = 0;
    const uint8_t *data = nullptr;
    int64_t rows() const { int64_t r = 1; for (size_t i = 1; i < dims.size(); i++) r *= dims[i]; return r; }
    int64_t cols() const { return dims.empty() ? 0 : dims[0]; }
};

struct GgufValue {
    int type = 0;            // GGUF value type
    int64_t i = 0;
    double f = 0.0;
    std::string s;
    std::vector<int64_t> ai;
    std::vector<double> af;
};

class Gguf {
public:
    // Open a file (mmap) or "mem:<name>" (an image from the registry). A
    // split model (<base>-%05d-of-%05d.gguf, split.no / split.count) opens
    // from any of its shards as one name→tensor map: shard 1 carries the
    // metadata, every shard its own tensor directory and data
    // (io/GgufFile.cajeta:45-55, :467-560).
    bool open(const std::string &path, std::string &err);
    int shards() const { return (int)maps_.size() > 0 ? (int)maps_.size() : 1; }
    ~Gguf();
    const GgufTensor *tensor(const std::string &name) const;
    bool has(const std::string &key) const { return kv_.count(key) != 0; }
    int64_t get_int(const std::string &key, int64_t dflt) const;
    double get_float(const std::string &key, double dflt) const;
    std::string get_str(const std::string &key, const std::string &dflt) const;
    const GgufValue *get(const std::string &key) const;
    const std::vector<GgufTensor> &tensors() const { return tensors_; }

private:
    // parse one file's header; metadata into kv (the model's for shard 1,
    // a scratch map for the others), tensors appended to the directory
    bool parse(const uint8_t *p, size_t n, std::map<std::string, GgufValue> &kv, std::string &err);
    bool map_file(const std::string &path, const uint8_t **p, size_t *n, std::string &err);
    std::map<std::string, GgufValue> kv_;
    std::vector<GgufTensor> tensors_;
    std::map<std::string, size_t> index_;
    std::vector<std::pair<void *, size_t>> maps_;
};

int64_t ggml_row_bytes(int type, int64_t cols);   // -1 when not whole blocks
int ggml_block_elems(int type);
int ggml_block_bytes(int type);

// Writer: metadata then tensor infos; data is filled in place afterwards.
class GgufWriter {
public:
    void kv_u32(const std::string &k, uint32_t v);
    void kv_i32(const std::string &k, int32_t v);
    void kv_f32(const std::string &k, float v);
    void kv_str(const std::string &k, const std::string &v);
    void kv_bool(const std::string &k, bool v);
    void tensor(const std::string &name, int type, std::vector<int64_t> dims);
    // Lay out the file; returns the total size and each tensor's byte offset
    // from the start of the image.
    size_t layout(std::vector<size_t> &offsets);
    // Write the header part (everything before the data) into `out`.
    void write_header(uint8_t *out) const;

private:
    std::vector<uint8_t> meta_;
    uint64_t n_kv_ = 0;
    struct T { std::string name; int type; std::vector<int64_t> dims; uint64_t off; int64_t bytes; };
    std::vector<T> ts_;
    size_t header_size_ = 0;
};

// In-process images ("mem:<name>"), owned by the registry.
uint8_t *image_create(const std::string &name, size_t bytes);
bool image_get(const std::string &name, const uint8_t **p, size_t *n);
bool image_free(const std::string &name);

}  // namespace cj
