// gguf.h -- GGUF v2/v3 container reader with the semantics of
// crates/gguf-rs/src/lib.rs:41-120 (header, metadata, tensor infos, aligned
// data start) and its rejection rules (lib.rs:127-332).
#pragma once

#include <cstdint>
#include <map>
#include <memory>
#include <string>
#include <vector>

namespace styx {

struct GgufValue {
    enum Kind { U8, I8, U16, I16, U32, I32, F32, BOOL, STR, ARR, U64, I64, F64 } kind = U32;
    uint64_t u = 0;  // unsigned / bool
    int64_t i = 0;   // signed
    double f = 0;    // f32 / f64
    std::string s;
    std::vector<GgufValue> arr;
};

struct GgufTensor {
    std::string name;
    std::vector<uint64_t> dims;
    uint32_t ggml_type = 0;
    uint64_t offset = 0;      // relative to data_start
    uint64_t size_bytes = 0;
};

struct Gguf {
    uint32_t version = 0;
    std::map<std::string, GgufValue> metadata;
    std::vector<GgufTensor> tensors;
    uint64_t data_start = 0;

    const GgufTensor *find(const std::string &name) const;
    bool get_u32(const std::string &key, uint32_t &out) const;
    bool get_f32(const std::string &key, float &out) const;
    bool get_str(const std::string &key, std::string &out) const;
};

// Parse the header of the file at `path`.  On failure returns false and sets
// err to a message that contains the reference's error text ("Invalid GGUF
// magic", "Unsupported GGUF version", "String too long", "Invalid UTF-8",
// "Unknown value type", "Array too long", "Unknown ggml_type",
// "First dimension not multiple of block size", or an I/O failure).
bool gguf_open(const std::string &path, Gguf &out, std::string &err);

// Block elements / bytes of a ggml type (lib.rs:242-332); false if unknown.
bool ggml_block(uint32_t type, uint64_t &elems, uint64_t &bytes);

}  // namespace styx
