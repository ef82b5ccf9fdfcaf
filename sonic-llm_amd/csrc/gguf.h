// GGUF v3 reader (mmap) and writer. The reader replaces the reference's gguf_open / tensor table (core.h:15-199);
// the writer produces the synthetic random-init models the configs name (the role of sllm-core's testutil.rs
// tiny_model writer, sllm-core/src/testutil.rs:22-162).
#pragma once
#include <stddef.h>
#include <stdint.h>

#include <map>
#include <string>
#include <vector>

enum GgmlType { GGML_F32 = 0, GGML_F16 = 1, GGML_Q4_0 = 2, GGML_Q8_0 = 8, GGML_Q6_K = 14 };

struct GgufValue {
    int type = -1;  // gguf value type of the scalar (or of the array's items)
    bool is_array = false;
    double num = 0;       // numeric scalars
    std::string str;      // strings
    uint64_t n_items = 0; // arrays (contents skipped)
};

struct GgufTensor {
    std::string name;
    int type = 0;
    int n_dims = 0;
    int64_t ne[4] = {1, 1, 1, 1};
    uint64_t offset = 0;   // from the data section
    const uint8_t* data = nullptr;
    size_t nbytes = 0;
};

struct GgufFile {
    int fd = -1;
    uint8_t* map = nullptr;
    size_t size = 0;
    uint32_t version = 0;
    size_t alignment = 32;
    size_t data_offset = 0;
    std::map<std::string, GgufValue> kv;
    std::vector<GgufTensor> tensors;
    std::map<std::string, size_t> index;

    bool open(const char* path, std::string* why);  // header, kv and tensor table; data stays mapped
    void close();
    ~GgufFile() { close(); }
    const GgufTensor* find(const std::string& name) const;
    double num(const std::string& key, double dflt) const;
    std::string str(const std::string& key) const;
};

size_t ggml_row_bytes(int type, int64_t ne0);

// ---- writer ----
struct GgufWriter {
    struct KV {
        std::string key;
        int type;  // 4 u32, 5 i32, 6 f32, 8 string
        double num;
        std::string str;
    };
    struct T {
        std::string name;
        int type;
        std::vector<int64_t> ne;
        size_t nbytes;
        uint64_t offset;
    };
    std::vector<KV> kvs;
    std::vector<T> ts;
    size_t alignment = 32;

    void u32(const std::string& k, uint32_t v) { kvs.push_back({k, 4, (double) v, ""}); }
    void f32(const std::string& k, float v) { kvs.push_back({k, 6, (double) v, ""}); }
    void str(const std::string& k, const std::string& v) { kvs.push_back({k, 8, 0, v}); }
    void tensor(const std::string& name, int type, std::vector<int64_t> ne);
    // writes header, kv, tensor table and alignment padding; returns the file offset of the data section
    bool begin(FILE* f, size_t* data_start);
};
