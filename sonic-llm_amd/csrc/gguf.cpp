#include "gguf.h"

#include <fcntl.h>
#include <stdio.h>
#include <string.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

size_t ggml_row_bytes(int type, int64_t ne0) {
    switch (type) {
        case GGML_F32: return (size_t) ne0 * 4;
        case GGML_F16: return (size_t) ne0 * 2;
        case GGML_Q4_0: return (size_t) (ne0 / 32) * 18;
        case GGML_Q8_0: return (size_t) (ne0 / 32) * 34;
        case GGML_Q6_K: return (size_t) (ne0 / 256) * 210;
        default: return 0;
    }
}

namespace {
struct Rd {
    const uint8_t* p;
    const uint8_t* end;
    bool ok = true;
    template <class T>
    T get() {
        T v{};
        if (sizeof(T) > (size_t) (end - p)) {
            ok = false;
            return v;
        }
        memcpy(&v, p, sizeof(T));
        p += sizeof(T);
        return v;
    }
    std::string s() {
        const uint64_t n = get<uint64_t>();
        if (!ok || n > (uint64_t) (end - p)) {
            ok = false;
            return {};
        }
        std::string r((const char*) p, n);
        p += n;
        return r;
    }
};
size_t scalar_size(int t) {
    switch (t) {
        case 0: case 1: case 7: return 1;
        case 2: case 3: return 2;
        case 4: case 5: case 6: return 4;
        case 10: case 11: case 12: return 8;
        default: return 0;
    }
}
double read_num(Rd& r, int t) {
    switch (t) {
        case 0: return r.get<uint8_t>();
        case 1: return r.get<int8_t>();
        case 2: return r.get<uint16_t>();
        case 3: return r.get<int16_t>();
        case 4: return r.get<uint32_t>();
        case 5: return r.get<int32_t>();
        case 6: return r.get<float>();
        case 7: return r.get<uint8_t>();
        case 10: return (double) r.get<uint64_t>();
        case 11: return (double) r.get<int64_t>();
        case 12: return r.get<double>();
        default: r.ok = false; return 0;
    }
}
}  // namespace

bool GgufFile::open(const char* path, std::string* why) {
    fd = ::open(path, O_RDONLY);
    if (fd < 0) {
        *why = std::string("cannot open ") + path;
        return false;
    }
    struct stat st;
    fstat(fd, &st);
    size = (size_t) st.st_size;
    map = (uint8_t*) mmap(nullptr, size, PROT_READ, MAP_PRIVATE, fd, 0);
    if (map == MAP_FAILED) {
        map = nullptr;
        *why = "mmap failed";
        return false;
    }
    Rd r{map, map + size};
    const uint32_t magic = r.get<uint32_t>();
    if (magic != 0x46554747u) {
        *why = "not a GGUF file";
        return false;
    }
    version = r.get<uint32_t>();
    if (version < 2 || version > 3) {
        *why = "unsupported GGUF version";
        return false;
    }
    const uint64_t n_t = r.get<uint64_t>(), n_kv = r.get<uint64_t>();
    for (uint64_t i = 0; i < n_kv && r.ok; ++i) {
        const std::string key = r.s();
        GgufValue v;
        v.type = (int) r.get<uint32_t>();
        if (v.type == 8) {
            v.str = r.s();
        } else if (v.type == 9) {
            v.is_array = true;
            const int it = (int) r.get<uint32_t>();
            v.n_items = r.get<uint64_t>();
            v.type = it;
            if (it == 8) {
                for (uint64_t j = 0; j < v.n_items && r.ok; ++j) r.s();
            } else {
                const size_t sz = scalar_size(it);
                if (!sz || v.n_items > (uint64_t) (r.end - r.p) / sz) r.ok = false;
                else r.p += sz * v.n_items;
            }
        } else {
            v.num = read_num(r, v.type);
        }
        kv[key] = v;
    }
    if (kv.count("general.alignment")) {
        // a power of two, at most 1 MiB (the data section starts at the next multiple of it)
        const double a = kv["general.alignment"].num;
        alignment = a >= 1 && a <= (1 << 20) ? (size_t) a : 0;
        if (!alignment || (alignment & (alignment - 1))) {
            *why = "general.alignment must be a power of two up to 1 MiB";
            return false;
        }
    }
    for (uint64_t i = 0; i < n_t && r.ok; ++i) {
        GgufTensor t;
        t.name = r.s();
        t.n_dims = (int) r.get<uint32_t>();
        if (t.n_dims < 1 || t.n_dims > 4) {
            r.ok = false;
            break;
        }
        for (int d = 0; d < t.n_dims; ++d) {
            const uint64_t ne = r.get<uint64_t>();
            if (ne < 1 || ne > (1ull << 40)) r.ok = false;  // (each factor of the size products below stays small)
            t.ne[d] = (int64_t) ne;
        }
        t.type = (int) r.get<uint32_t>();
        t.offset = r.get<uint64_t>();
        tensors.push_back(t);
    }
    if (!r.ok) {
        *why = "truncated or malformed GGUF header";
        return false;
    }
    const size_t hdr = (size_t) (r.p - map);
    data_offset = (hdr + alignment - 1) / alignment * alignment;
    if (data_offset > size) {
        *why = "truncated GGUF file (no data section)";
        return false;
    }
    const size_t room = size - data_offset;  // bytes of the data section
    for (size_t i = 0; i < tensors.size(); ++i) {
        GgufTensor& t = tensors[i];
        const size_t rb = ggml_row_bytes(t.type, t.ne[0]);
        const int bk = t.type == GGML_Q6_K ? 256 : (t.type == GGML_Q4_0 || t.type == GGML_Q8_0) ? 32 : 1;
        // rows: each dimension at most 2^40 (checked above), so every partial product is checked against the room
        // before the next multiply
        size_t rows = 1;
        bool fits = rb != 0 && t.ne[0] % bk == 0;
        for (int d = 1; d < 4 && fits; ++d) {
            if ((size_t) t.ne[d] > room / rows) fits = false;
            else rows *= (size_t) t.ne[d];
        }
        fits = fits && rows <= room / rb;
        t.nbytes = fits ? rb * rows : 0;
        if (!fits || t.offset > room || t.nbytes > room - t.offset) {
            *why = "tensor " + t.name + ": unsupported type or shape, or out of the file";
            return false;
        }
        t.data = map + data_offset + t.offset;
        index[t.name] = i;
    }
    return true;
}

void GgufFile::close() {
    if (map) munmap(map, size);
    if (fd >= 0) ::close(fd);
    map = nullptr;
    fd = -1;
}

const GgufTensor* GgufFile::find(const std::string& name) const {
    auto it = index.find(name);
    return it == index.end() ? nullptr : &tensors[it->second];
}

double GgufFile::num(const std::string& key, double dflt) const {
    auto it = kv.find(key);
    return it == kv.end() || it->second.is_array || it->second.type == 8 ? dflt : it->second.num;
}

std::string GgufFile::str(const std::string& key) const {
    auto it = kv.find(key);
    return it == kv.end() ? std::string() : it->second.str;
}

void GgufWriter::tensor(const std::string& name, int type, std::vector<int64_t> ne) {
    size_t rows = 1;
    for (size_t i = 1; i < ne.size(); ++i) rows *= (size_t) ne[i];
    T t{name, type, ne, ggml_row_bytes(type, ne[0]) * rows, 0};
    uint64_t off = 0;
    if (!ts.empty()) {
        off = ts.back().offset + ts.back().nbytes;
        off = (off + alignment - 1) / alignment * alignment;
    }
    t.offset = off;
    ts.push_back(t);
}

bool GgufWriter::begin(FILE* f, size_t* data_start) {
    auto w = [&](const void* p, size_t n) { return fwrite(p, 1, n, f) == n; };
    auto ws = [&](const std::string& s) {
        const uint64_t n = s.size();
        return w(&n, 8) && w(s.data(), n);
    };
    const uint32_t magic = 0x46554747u, version = 3;
    const uint64_t nt = ts.size(), nkv = kvs.size();
    bool ok = w(&magic, 4) && w(&version, 4) && w(&nt, 8) && w(&nkv, 8);
    for (const KV& k : kvs) {
        const uint32_t t = (uint32_t) k.type;
        ok = ok && ws(k.key) && w(&t, 4);
        if (k.type == 8) ok = ok && ws(k.str);
        else if (k.type == 6) { const float v = (float) k.num; ok = ok && w(&v, 4); }
        else if (k.type == 5) { const int32_t v = (int32_t) k.num; ok = ok && w(&v, 4); }
        else { const uint32_t v = (uint32_t) k.num; ok = ok && w(&v, 4); }
    }
    for (const T& t : ts) {
        const uint32_t nd = (uint32_t) t.ne.size(), ty = (uint32_t) t.type;
        ok = ok && ws(t.name) && w(&nd, 4);
        for (int64_t e : t.ne) { const uint64_t v = (uint64_t) e; ok = ok && w(&v, 8); }
        ok = ok && w(&ty, 4) && w(&t.offset, 8);
    }
    long pos = ftell(f);
    const size_t start = ((size_t) pos + alignment - 1) / alignment * alignment;
    static const uint8_t zeros[64] = {0};
    for (size_t left = start - (size_t) pos; ok && left > 0;) {  // (alignments above 64 bytes: in pieces)
        const size_t n = left < sizeof zeros ? left : sizeof zeros;
        ok = w(zeros, n);
        left -= n;
    }
    *data_start = start;
    return ok;
}
