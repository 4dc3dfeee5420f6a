// gguf.cpp - bounds-checked GGUF reader (see gguf.h).
#include "gguf.h"
#include "common.h"

#include <cinttypes>
#include <cstring>
#include <memory>
#include <sstream>

type_traits ggml_traits(int type) {
    switch (type) {
        case T_F32:  return {1, 4, "f32"};
        case T_F16:  return {1, 2, "f16"};
        case T_BF16: return {1, 2, "bf16"};
        case T_Q4_0: return {32, 18, "q4_0"};
        case T_Q4_1: return {32, 20, "q4_1"};
        case T_Q5_0: return {32, 22, "q5_0"};
        case T_Q5_1: return {32, 24, "q5_1"};
        case T_Q8_0: return {32, 34, "q8_0"};
        case T_Q8_1: return {32, 36, "q8_1"};
        case T_Q2_K: return {256, 84, "q2_K"};
        case T_Q3_K: return {256, 110, "q3_K"};
        case T_Q4_K: return {256, 144, "q4_K"};
        case T_Q5_K: return {256, 176, "q5_K"};
        case T_Q6_K: return {256, 210, "q6_K"};
        case T_Q8_K: return {256, 292, "q8_K"};
        default:     return {0, 0, "unknown"};
    }
}

namespace gguf {

namespace {

struct reader {
    FILE * f;
    uint64_t size;
    uint64_t pos = 0;
    std::string err;

    bool bytes(void * dst, uint64_t n) {
        if (n > size || pos > size - n) { err = "unexpected end of file"; return false; }
        if (fread(dst, 1, (size_t) n, f) != n) { err = "short read"; return false; }
        pos += n;
        return true;
    }
    template <typename T> bool get(T & v) { return bytes(&v, sizeof(T)); }
    bool str(std::string & s) {
        uint64_t n = 0;
        if (!get(n)) return false;
        if (n > (1u << 24) || n > size - pos) { err = "string length out of range"; return false; }
        s.resize((size_t) n);
        return n == 0 || bytes(&s[0], n);
    }
};

bool scalar(reader & r, uint32_t t, value & v) {
    v.type = t;
    switch (t) {
        case U8:   { uint8_t x;  if (!r.get(x)) return false; v.i = x; v.f = x; return true; }
        case I8:   { int8_t x;   if (!r.get(x)) return false; v.i = x; v.f = x; return true; }
        case U16:  { uint16_t x; if (!r.get(x)) return false; v.i = x; v.f = x; return true; }
        case I16:  { int16_t x;  if (!r.get(x)) return false; v.i = x; v.f = x; return true; }
        case U32:  { uint32_t x; if (!r.get(x)) return false; v.i = x; v.f = x; return true; }
        case I32:  { int32_t x;  if (!r.get(x)) return false; v.i = x; v.f = x; return true; }
        case U64:  { uint64_t x; if (!r.get(x)) return false; v.i = (int64_t) x; v.f = (double) x; return true; }
        case I64:  { int64_t x;  if (!r.get(x)) return false; v.i = x; v.f = (double) x; return true; }
        case F32:  { float x;    if (!r.get(x)) return false; v.f = x; v.i = (int64_t) x; return true; }
        case F64:  { double x;   if (!r.get(x)) return false; v.f = x; v.i = (int64_t) x; return true; }
        case BOOL: { uint8_t x;  if (!r.get(x)) return false; v.i = x != 0; v.f = v.i; return true; }
        case STR:  return r.str(v.s);
        default: r.err = "unknown metadata value type " + std::to_string(t); return false;
    }
}

}  // namespace

std::string value::render() const {
    std::ostringstream os;
    switch (type) {
        case STR: os << '"' << s << '"'; break;
        case F32: case F64: os << f; break;
        case BOOL: os << (i ? "true" : "false"); break;
        case ARR: {
            os << '[';
            const size_t n = arr_type == STR ? as.size() : af.size();
            for (size_t k = 0; k < n && k < 16; k++) {
                if (k) os << ", ";
                if (arr_type == STR) os << '"' << as[k] << '"'; else os << af[k];
            }
            if (n > 16) os << ", ... (" << n << " items)";
            os << ']';
            break;
        }
        default: os << i;
    }
    return os.str();
}

const value * file::find(const std::string & key) const {
    for (const auto & p : kv) if (p.first == key) return &p.second;
    return nullptr;
}

const tensor_info * file::tensor(const std::string & name) const {
    for (const auto & t : tensors) if (t.name == name) return &t;
    return nullptr;
}

bool open(const std::string & path, file & out, std::string & err) {
    std::unique_ptr<FILE, int (*)(FILE *)> fp(fopen(path.c_str(), "rb"), fclose);
    if (!fp) { err = "cannot open " + path; return false; }
    if (fseeko(fp.get(), 0, SEEK_END) != 0) { err = "cannot seek " + path; return false; }
    const int64_t fsz = (int64_t) ftello(fp.get());
    fseeko(fp.get(), 0, SEEK_SET);
    if (fsz < 24) { err = path + " is too small to be a GGUF file"; return false; }
    reader r{fp.get(), (uint64_t) fsz};
    char magic[4];
    uint32_t version = 0;
    uint64_t n_tensors = 0, n_kv = 0;
    if (!r.bytes(magic, 4) || memcmp(magic, "GGUF", 4) != 0) { err = path + ": bad magic (not a GGUF file)"; return false; }
    if (!r.get(version) || (version != 2 && version != 3)) { err = path + ": unsupported GGUF version " + std::to_string(version); return false; }
    if (!r.get(n_tensors) || !r.get(n_kv)) { err = path + ": " + r.err; return false; }
    // every kv takes at least 12 bytes and every tensor info at least 24: cheap sanity bounds
    if (n_kv > (uint64_t) fsz / 12 || n_tensors > (uint64_t) fsz / 24) { err = path + ": header counts exceed the file size"; return false; }
    out = file();
    out.path = path;
    out.file_size = (uint64_t) fsz;
    uint64_t alignment = 32;
    for (uint64_t i = 0; i < n_kv; i++) {
        const uint64_t kv_begin = r.pos;
        std::string key;
        uint32_t t = 0;
        if (!r.str(key) || !r.get(t)) { err = path + ": " + r.err; return false; }
        value v;
        if (t == ARR) {
            uint32_t et = 0;
            uint64_t n = 0;
            if (!r.get(et) || !r.get(n)) { err = path + ": " + r.err; return false; }
            if (n > (uint64_t) fsz) { err = path + ": array length out of range for " + key; return false; }
            v.type = ARR;
            v.arr_type = et;
            for (uint64_t k = 0; k < n; k++) {
                value e;
                if (et == ARR || !scalar(r, et, e)) { err = path + ": bad array element in " + key + (r.err.empty() ? "" : ": " + r.err); return false; }
                if (et == STR) v.as.push_back(e.s);
                else { v.ai.push_back(e.i); v.af.push_back(e.f); }
            }
        } else if (!scalar(r, t, v)) {
            err = path + ": bad value for " + key + ": " + r.err;
            return false;
        }
        if (key == "general.alignment") {
            if (v.i <= 0 || v.i > 65536 || (v.i & (v.i - 1))) { err = path + ": general.alignment is not a power of two"; return false; }
            alignment = (uint64_t) v.i;
        }
        out.kv.emplace_back(key, std::move(v));
        out.kv_span.emplace_back(kv_begin, r.pos);
    }
    for (uint64_t i = 0; i < n_tensors; i++) {
        tensor_info ti;
        uint32_t nd = 0, ty = 0;
        if (!r.str(ti.name) || !r.get(nd)) { err = path + ": " + r.err; return false; }
        if (nd < 1 || nd > 4) { err = path + ": tensor " + ti.name + " has " + std::to_string(nd) + " dimensions"; return false; }
        ti.n_dims = (int) nd;
        int64_t nel = 1;
        for (uint32_t d = 0; d < nd; d++) {
            uint64_t v = 0;
            if (!r.get(v)) { err = path + ": " + r.err; return false; }
            if (v == 0 || v > (1ull << 40)) { err = path + ": tensor " + ti.name + " has a dimension of " + std::to_string(v); return false; }
            ti.ne[d] = (int64_t) v;
            if (nel > (int64_t) (1ull << 42) / (int64_t) v) { err = path + ": tensor " + ti.name + " is too large"; return false; }
            nel *= (int64_t) v;
        }
        uint64_t off = 0;
        if (!r.get(ty) || !r.get(off)) { err = path + ": " + r.err; return false; }
        ti.type = (int) ty;
        const type_traits tt = ggml_traits(ti.type);
        if (tt.blck == 0) { err = path + ": tensor " + ti.name + " has unsupported dtype " + std::to_string(ty); return false; }
        if (ti.ne[0] % tt.blck != 0) { err = path + ": tensor " + ti.name + " row is not a whole number of blocks"; return false; }
        ti.nbytes = (uint64_t) (nel / tt.blck) * (uint64_t) tt.bytes;
        ti.offset = off;
        out.tensors.push_back(std::move(ti));
    }
    const uint64_t data0 = (r.pos + alignment - 1) / alignment * alignment;
    out.data_offset = data0;
    for (auto & t : out.tensors) {
        const uint64_t abs = data0 + t.offset;
        if (t.offset > (uint64_t) fsz || abs > (uint64_t) fsz || t.nbytes > (uint64_t) fsz - abs) {
            char buf[256];
            snprintf(buf, sizeof(buf), "tensor %s claims %" PRIu64 " bytes at offset %" PRIu64 ", past the end of the file (%" PRId64 " bytes)",
                     t.name.c_str(), t.nbytes, abs, fsz);
            err = path + ": " + buf;
            return false;
        }
        t.offset = abs;
    }
    return true;
}

}  // namespace gguf
