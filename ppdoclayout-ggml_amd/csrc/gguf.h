// Minimal GGUF (v2/v3) reader for F32 model files, as written by the
// reference's converter (scripts/convert.py): header, key/value metadata,
// tensor infos, aligned data section.  Only what loading needs is kept:
// general.alignment, integer/string metadata, and each tensor's name, dims
// (ggml ne order), type and file offset.
#pragma once

#include <cstdint>
#include <map>
#include <string>
#include <vector>

namespace ppdl {

struct GgufTensor {
    std::string name;
    std::vector<int64_t> ne;  // ggml order: ne[0] fastest
    uint32_t type = 0;        // ggml_type (0 = F32)
    uint64_t offset = 0;      // absolute file offset of the data
    int64_t nelem() const {
        int64_t n = 1;
        for (int64_t d : ne) n *= d;
        return n;
    }
};

struct GgufFile {
    std::string path;
    uint32_t version = 0;
    uint64_t alignment = 32;
    std::map<std::string, int64_t> ints;
    std::map<std::string, std::string> strings;
    std::vector<GgufTensor> tensors;
    std::map<std::string, size_t> index;  // name -> tensors[i]
};

// Parses the header and tensor table.  Returns false (and fills *err) on a
// malformed or unsupported file.
bool gguf_open(const std::string &path, GgufFile *out, std::string *err);
// Reads one F32 tensor's data into dst (nelem floats).
bool gguf_read_f32(const GgufFile &f, const GgufTensor &t, float *dst, std::string *err);

}  // namespace ppdl
