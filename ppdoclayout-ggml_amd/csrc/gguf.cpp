// GGUF reader (see gguf.h).  Format: "GGUF", u32 version, u64 n_tensors,
// u64 n_kv; n_kv x (string key, u32 type, value); n_tensors x (string name,
// u32 n_dims, u64 ne[n_dims], u32 ggml_type, u64 offset); padding to
// general.alignment; data.  Strings are u64 length + bytes.
#include "gguf.h"

#include <cstdio>
#include <cstring>

namespace ppdl {
namespace {

enum : uint32_t {
    T_U8 = 0, T_I8 = 1, T_U16 = 2, T_I16 = 3, T_U32 = 4, T_I32 = 5, T_F32 = 6, T_BOOL = 7,
    T_STR = 8, T_ARR = 9, T_U64 = 10, T_I64 = 11, T_F64 = 12
};

struct Reader {
    FILE *f;
    bool ok = true;
    template <class T>
    T get() {
        T v{};
        if (ok && fread(&v, sizeof(T), 1, f) != 1) ok = false;
        return v;
    }
    std::string str() {
        const uint64_t n = get<uint64_t>();
        if (!ok || n > (1u << 20)) {
            ok = false;
            return {};
        }
        std::string s(n, '\0');
        if (n && fread(&s[0], 1, n, f) != n) ok = false;
        return s;
    }
    void skip(uint64_t n) {
        if (ok && fseeko(f, (off_t)n, SEEK_CUR) != 0) ok = false;
    }
};

int scalar_size(uint32_t t) {
    switch (t) {
        case T_U8: case T_I8: case T_BOOL: return 1;
        case T_U16: case T_I16: return 2;
        case T_U32: case T_I32: case T_F32: return 4;
        case T_U64: case T_I64: case T_F64: return 8;
        default: return 0;
    }
}

bool read_int(Reader &r, uint32_t t, int64_t *v) {
    switch (t) {
        case T_U8: *v = r.get<uint8_t>(); return true;
        case T_I8: *v = r.get<int8_t>(); return true;
        case T_U16: *v = r.get<uint16_t>(); return true;
        case T_I16: *v = r.get<int16_t>(); return true;
        case T_U32: *v = r.get<uint32_t>(); return true;
        case T_I32: *v = r.get<int32_t>(); return true;
        case T_U64: *v = (int64_t)r.get<uint64_t>(); return true;
        case T_I64: *v = r.get<int64_t>(); return true;
        case T_BOOL: *v = r.get<uint8_t>(); return true;
        default: return false;
    }
}

}  // namespace

bool gguf_open(const std::string &path, GgufFile *out, std::string *err) {
    FILE *f = fopen(path.c_str(), "rb");
    if (!f) {
        *err = "cannot open " + path;
        return false;
    }
    Reader r{f};
    char magic[4];
    if (fread(magic, 1, 4, f) != 4 || memcmp(magic, "GGUF", 4) != 0) {
        fclose(f);
        *err = "not a GGUF file: " + path;
        return false;
    }
    GgufFile g;
    g.path = path;
    g.version = r.get<uint32_t>();
    if (g.version < 2 || g.version > 3) {
        fclose(f);
        *err = "unsupported GGUF version " + std::to_string(g.version);
        return false;
    }
    const uint64_t n_tensors = r.get<uint64_t>(), n_kv = r.get<uint64_t>();
    for (uint64_t i = 0; r.ok && i < n_kv; i++) {
        const std::string key = r.str();
        const uint32_t t = r.get<uint32_t>();
        int64_t iv;
        if (t == T_STR) {
            g.strings[key] = r.str();
        } else if (t == T_ARR) {
            const uint32_t et = r.get<uint32_t>();
            const uint64_t n = r.get<uint64_t>();
            if (et == T_STR) {
                for (uint64_t j = 0; r.ok && j < n; j++) r.str();
            } else {
                const int sz = scalar_size(et);
                if (!sz) r.ok = false;
                r.skip(n * (uint64_t)sz);
            }
        } else if (read_int(r, t, &iv)) {
            g.ints[key] = iv;
        } else if (t == T_F32) {
            r.get<float>();
        } else if (t == T_F64) {
            r.get<double>();
        } else {
            r.ok = false;
        }
    }
    if (g.ints.count("general.alignment")) g.alignment = (uint64_t)g.ints["general.alignment"];
    if (g.alignment == 0 || (g.alignment & (g.alignment - 1))) r.ok = false;
    for (uint64_t i = 0; r.ok && i < n_tensors; i++) {
        GgufTensor t;
        t.name = r.str();
        const uint32_t nd = r.get<uint32_t>();
        if (nd > 4) r.ok = false;
        for (uint32_t d = 0; r.ok && d < nd; d++) t.ne.push_back((int64_t)r.get<uint64_t>());
        t.type = r.get<uint32_t>();
        t.offset = r.get<uint64_t>();
        g.index[t.name] = g.tensors.size();
        g.tensors.push_back(t);
    }
    if (!r.ok) {
        fclose(f);
        *err = "truncated or malformed GGUF: " + path;
        return false;
    }
    const uint64_t pos = (uint64_t)ftello(f);
    const uint64_t data = (pos + g.alignment - 1) / g.alignment * g.alignment;
    fseeko(f, 0, SEEK_END);
    const uint64_t size = (uint64_t)ftello(f);
    fclose(f);
    for (auto &t : g.tensors) {
        t.offset += data;
        const uint64_t bytes = (uint64_t)t.nelem() * 4;
        if (t.type == 0 && t.offset + bytes > size) {
            *err = "tensor " + t.name + " runs past the end of " + path;
            return false;
        }
    }
    *out = std::move(g);
    return true;
}

bool gguf_read_f32(const GgufFile &g, const GgufTensor &t, float *dst, std::string *err) {
    if (t.type != 0) {
        *err = "tensor " + t.name + " is not F32";
        return false;
    }
    FILE *f = fopen(g.path.c_str(), "rb");
    if (!f) {
        *err = "cannot open " + g.path;
        return false;
    }
    const size_t n = (size_t)t.nelem();
    const bool ok = fseeko(f, (off_t)t.offset, SEEK_SET) == 0 && fread(dst, 4, n, f) == n;
    fclose(f);
    if (!ok) *err = "short read of " + t.name;
    return ok;
}

}  // namespace ppdl
