// okf_gguf.h -- host side of the weight path: a GGUF file mapped read-only,
// its key/value metadata and tensor directory parsed with bounds checks, and
// its tensor data made resident in device memory.
//
// Follows GGUF(path:) (LLM/Base/GGUF.swift:99-151): magic "GGUF", version,
// tensor and key counts, typed key/values (general.alignment, default 32,
// sets the data alignment), then per tensor name, dims (ggml order), type
// and offset; the data region starts at the first aligned byte after the
// directory.  Byte sizes are GGUF.rowByteCount (GGUF.swift:160-188).  Where
// the reference traps on a malformed file (precondition / fatalError) this
// returns OKF_E_FORMAT.
#pragma once
#include <fcntl.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <cstdint>
#include <cstring>
#include <string>
#include <unordered_map>
#include <vector>

namespace okf_gguf_impl {

// GGUF.rowByteCount for every type id of GGUFType (GGUF.swift:3-14); 0 for an
// id that is not one of them.
inline uint64_t row_bytes(int32_t t, uint64_t n) {
    switch (t) {
    case 0: return n * 4;                // f32
    case 1: case 30: return n * 2;       // f16, bf16
    case 42: return n / 128 * 34;        // q2_0
    case 41: return n / 128 * 18;        // q1_0
    case 10: return n / 256 * 84;        // q2_k
    case 11: return n / 256 * 110;       // q3_k
    case 12: return n / 256 * 144;       // q4_k
    case 13: return n / 256 * 176;       // q5_k
    case 14: return n / 256 * 210;       // q6_k
    case 15: return n / 256 * 292;       // q8_k
    case 16: return n / 256 * 66;        // iq2_xxs
    case 17: return n / 256 * 74;        // iq2_xs
    case 22: return n / 256 * 82;        // iq2_s
    case 18: return n / 256 * 98;        // iq3_xxs
    case 21: return n / 256 * 110;       // iq3_s
    case 23: return n / 256 * 136;       // iq4_xs
    case 20: return n / 32 * 18;         // iq4_nl
    case 19: return n / 256 * 50;        // iq1_s
    case 29: return n / 256 * 56;        // iq1_m
    case 2: return n / 32 * 18;          // q4_0
    case 3: return n / 32 * 20;          // q4_1
    case 6: return n / 32 * 22;          // q5_0
    case 7: return n / 32 * 24;          // q5_1
    case 8: return n / 32 * 34;          // q8_0
    case 9: return n / 32 * 36;          // q8_1
    default: return 0;
    }
}

struct Value {
    enum Kind { Int, Double, String, Ints, Doubles, Strings, Bool } kind = Int;
    int64_t i = 0;
    double d = 0;
    std::string s;
    std::vector<int64_t> is;
    std::vector<double> ds;
    std::vector<std::string> ss;
};

struct Tensor {
    std::string name;
    uint32_t n_dims = 0;
    uint64_t dims[4] = {1, 1, 1, 1};
    int32_t type = 0;
    uint64_t offset = 0, bytes = 0;
};

struct File {
    int fd = -1;
    const uint8_t *map = nullptr;
    uint64_t size = 0;
    uint64_t data_start = 0;
    std::unordered_map<std::string, Value> meta;
    std::vector<Tensor> tensors;
    std::unordered_map<std::string, size_t> by_name;
    ~File() {
        if (map) munmap((void *)map, size);
        if (fd >= 0) close(fd);
    }
};

// Bounds-checked little-endian reader over the mapping.
struct Cursor {
    const uint8_t *p;
    uint64_t size, pos = 0;
    bool ok = true;
    const uint8_t *take(uint64_t n) {
        if (!ok || n > size - pos) {
            ok = false;
            return nullptr;
        }
        const uint8_t *r = p + pos;
        pos += n;
        return r;
    }
    template <class T>
    T get() {
        T v{};
        if (const uint8_t *q = take(sizeof(T))) std::memcpy(&v, q, sizeof(T));
        return v;
    }
    std::string str() {
        const uint64_t n = get<uint64_t>();
        const uint8_t *q = take(n);
        return q ? std::string((const char *)q, n) : std::string();
    }
};

// One scalar of GGUF value type t (GGUF.swift:326-344).
inline bool scalar(Cursor &c, uint32_t t, Value &v) {
    switch (t) {
    case 0: v.kind = Value::Int; v.i = c.get<uint8_t>(); return true;
    case 1: v.kind = Value::Int; v.i = c.get<int8_t>(); return true;
    case 2: v.kind = Value::Int; v.i = c.get<uint16_t>(); return true;
    case 3: v.kind = Value::Int; v.i = c.get<int16_t>(); return true;
    case 4: v.kind = Value::Int; v.i = c.get<uint32_t>(); return true;
    case 5: v.kind = Value::Int; v.i = c.get<int32_t>(); return true;
    case 6: v.kind = Value::Double; v.d = c.get<float>(); return true;
    case 7: v.kind = Value::Bool; v.i = c.get<uint8_t>() != 0; return true;
    case 8: v.kind = Value::String; v.s = c.str(); return true;
    case 10: v.kind = Value::Int; v.i = (int64_t)c.get<uint64_t>(); return true;
    case 11: v.kind = Value::Int; v.i = c.get<int64_t>(); return true;
    case 12: v.kind = Value::Double; v.d = c.get<double>(); return true;
    default: return false;
    }
}

// A typed value; arrays as in GGUF.swift:347-368 (strings kept as strings,
// bools as ints, any float element makes the array doubles).
inline bool value(Cursor &c, Value &v) {
    const uint32_t t = c.get<uint32_t>();
    if (t != 9) return scalar(c, t, v);
    const uint32_t et = c.get<uint32_t>();
    const uint64_t n = c.get<uint64_t>();
    if (!c.ok || et == 9 || n > c.size) return false;  // every element takes >= 1 byte
    if (et == 8) {
        v.kind = Value::Strings;
        for (uint64_t k = 0; k < n && c.ok; k++) v.ss.push_back(c.str());
        return c.ok;
    }
    bool dbl = false;
    for (uint64_t k = 0; k < n && c.ok; k++) {
        Value e;
        if (!scalar(c, et, e)) return false;
        if (e.kind == Value::Double) {
            dbl = true;
            v.ds.push_back(e.d);
        } else {
            v.is.push_back(e.i);
        }
    }
    v.kind = dbl ? Value::Doubles : Value::Ints;
    return c.ok;
}

// 0 = ok, 7 = io, 8 = format (the status codes of okf_quant.h)
inline int parse(File &f) {
    Cursor c{f.map, f.size};
    if (c.get<uint32_t>() != 0x46554747u) return 8;  // "GGUF"
    (void)c.get<uint32_t>();                          // version
    const uint64_t nt = c.get<uint64_t>(), nkv = c.get<uint64_t>();
    if (!c.ok || nt > f.size || nkv > f.size) return 8;
    uint64_t alignment = 32;
    for (uint64_t k = 0; k < nkv; k++) {
        std::string key = c.str();
        Value v;
        if (!value(c, v) || !c.ok) return 8;
        if (key == "general.alignment" && v.kind == Value::Int) {
            // a power of two up to 1 MiB (GGUF requires a power of two)
            if (v.i <= 0 || v.i > (1 << 20) || (v.i & (v.i - 1))) return 8;
            alignment = (uint64_t)v.i;
        }
        f.meta[key] = std::move(v);
    }
    for (uint64_t k = 0; k < nt; k++) {
        Tensor t;
        t.name = c.str();
        t.n_dims = c.get<uint32_t>();
        if (!c.ok || t.n_dims > 4) return 8;
        uint64_t n = 1;
        for (uint32_t d = 0; d < t.n_dims; d++) {
            t.dims[d] = c.get<uint64_t>();
            if (__builtin_mul_overflow(n, t.dims[d], &n)) return 8;
        }
        if (n > (1ull << 60)) return 8;  // (so that row_bytes cannot wrap)
        t.type = (int32_t)c.get<uint32_t>();
        t.offset = c.get<uint64_t>();
        if (!c.ok) return 8;
        t.bytes = row_bytes(t.type, n);
        if (t.bytes == 0 && n != 0) return 8;  // not a GGUFType
        f.by_name[t.name] = f.tensors.size();
        f.tensors.push_back(std::move(t));
    }
    f.data_start = (c.pos + alignment - 1) / alignment * alignment;
    if (f.data_start > f.size) return 8;  // (also with no tensors)
    for (const Tensor &t : f.tensors)
        if (t.offset > f.size - f.data_start || t.bytes > f.size - f.data_start - t.offset)
            return 8;  // tensor past the end of the file
    return 0;
}

}  // namespace okf_gguf_impl
