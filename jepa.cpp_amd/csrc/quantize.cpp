// quantize.cpp - jepa_amd_quantize_file: re-type the weights of a jepa GGUF (reference
// tools/jepa-quantize.cpp), with the block quantization on the GPU (quant.hip).
//
// The rule, the plan and the output file follow the reference tool:
//   - only 2-D `.weight` matrices of the attention / FFN / projection / classifier layers change type
//     (tools/jepa-quantize.cpp:90-129), minus the caller's keep list; target f32 widens every tensor;
//   - a K-quant whose row length is not a multiple of 256 falls back per tensor to q4_0, and a tensor
//     whose rows are not whole blocks of the target keeps its type (:371-387);
//   - an already-quantized tensor is re-quantized only when allowed (:362-369);
//   - every metadata pair is copied verbatim and in order, general.file_type takes the target's ftype
//     in place (appended when absent), general.alignment is dropped and the default 32 used (:302-318);
//     when fallbacks leave most quantized tensors in another type, file_type names that type and,
//     as the reference's gguf_set_val_u32 does, moves to the end (:409-431);
//   - tensor infos keep the input order with trailing unit dimensions trimmed, data offsets aligned
//     to 32, and every tensor's data zero-padded to 32 (ggml's GGUF v3 writer).
// Types: f32, f16, q8_0, q4_0 and q4_k (the ones this library's GEMMs run); the reference's other
// targets (q4_1, q5_0, q5_1, q5_k, q6_k) are refused with a message.
#include "../../include/jepa_amd.h"
#include "common.h"
#include "gguf.h"
#include "kernels.h"

#include <hip/hip_runtime.h>

#include <algorithm>
#include <cctype>
#include <cinttypes>
#include <cstdio>
#include <cstring>
#include <map>
#include <memory>
#include <string>
#include <vector>

namespace {

struct target_spec { const char * name; int type; uint32_t ftype; };
// TYPE name -> tensor type and the general.file_type (ggml ftype) the reference tool writes for it
// (tools/jepa-quantize.cpp:41-52, docs/quantization.md:29-31)
const target_spec TARGETS[] = {
    {"f32", T_F32, 0}, {"f16", T_F16, 1}, {"q8_0", T_Q8_0, 7}, {"q4_0", T_Q4_0, 2}, {"q4_k", T_Q4_K, 12},
};

bool is_quantized(int t) { return ggml_traits(t).blck > 1; }

bool contains(const std::string & s, const char * sub) { return s.find(sub) != std::string::npos; }
bool starts_with(const std::string & s, const char * pre) { return s.rfind(pre, 0) == 0; }

// reference tools/jepa-quantize.cpp:90-129
bool is_quantizable(const std::string & name, int n_dims) {
    if (n_dims != 2 || name.size() < 7 || name.compare(name.size() - 7, 7, ".weight") != 0) return false;
    static const char * const KEEP[] = {"patch_embed", "pos_embed", "cls_token", "reg_tokens", "mask_tokens", "mod_embed", ".adaln.",
                                        "action_embed", "state_embed", ".ln1.", ".ln2.", ".norm.", "hier_norm", "ln_kv", "head.query",
                                        ".act_enc.", ".act_embed.", "act_queue"};
    for (const char * k : KEEP) if (contains(name, k)) return false;
    static const char * const COMPONENTS[] = {".attn_qkv.", ".attn_q.", ".attn_k.", ".attn_v.", ".attn_out.", ".ffn_up.", ".ffn_down."};
    for (const char * c : COMPONENTS) if (contains(name, c)) return true;
    static const char * const PREFIXES[] = {"pred.proj", "pred.embed", "enc.proj.", "head.cls.", "head.xattn."};
    for (const char * p : PREFIXES) if (starts_with(name, p)) return true;
    static const char * const LEVEL_PARTS[] = {".enc.proj.", ".enc.fc1.", ".enc.fc2.", ".pred.proj.", ".pred.in_proj.", ".pred.cond_proj.",
                                               ".pred.out_proj."};
    if (starts_with(name, "lvl."))
        for (const char * c : LEVEL_PARTS) if (contains(name, c)) return true;
    return false;
}

struct plan_item {
    const gguf::tensor_info * t = nullptr;
    int n_dims = 1;
    int dst = T_F32;
    uint64_t dst_bytes = 0, dst_offset = 0;
    std::string note;
};

uint64_t pad32(uint64_t n) { return (n + 31) / 32 * 32; }

struct writer {
    FILE * f = nullptr;
    bool ok = true;
    void bytes(const void * p, size_t n) { if (ok && n && fwrite(p, 1, n, f) != n) ok = false; }
    template <typename T> void put(T v) { bytes(&v, sizeof(T)); }
    void str(const std::string & s) { put<uint64_t>(s.size()); bytes(s.data(), s.size()); }
    void zeros(size_t n) { static const uint8_t z[64] = {0}; while (n) { const size_t k = std::min<size_t>(n, 64); bytes(z, k); n -= k; } }
};

struct dev_buf {
    void * p = nullptr;
    size_t cap = 0;
    ~dev_buf() { if (p) hipFree(p); }
    bool need(size_t n) {
        if (n <= cap) return true;
        if (p) hipFree(p);
        p = nullptr; cap = 0;
        if (hipMalloc(&p, n) != hipSuccess) return false;
        cap = n;
        return true;
    }
};

}  // namespace

extern "C" int jepa_amd_quantize_file(const char * in_path, const char * out_path, const char * type, const char * const * keep, int n_keep,
                                      bool allow_requant, int device, bool verbose) {
    if (!in_path || !out_path || !type || (n_keep > 0 && !keep)) return -1;
    std::string tl = type;
    std::transform(tl.begin(), tl.end(), tl.begin(), [](unsigned char c) { return (char) std::tolower(c); });
    const target_spec * spec = nullptr;
    for (const auto & t : TARGETS) if (tl == t.name) spec = &t;
    if (!spec) {
        const bool ref_type = tl == "q4_1" || tl == "q5_0" || tl == "q5_1" || tl == "q5_k" || tl == "q6_k";
        jepa_log("jepa: jepa_amd_quantize_file: %s type '%s' (f32, f16, q8_0, q4_0 or q4_k)\n", ref_type ? "this library does not write" : "unknown",
                 type);
        return -1;
    }
    if (strcmp(in_path, out_path) == 0) { jepa_log("jepa: jepa_amd_quantize_file: IN and OUT must differ\n"); return -1; }
    gguf::file in;
    std::string err;
    if (!gguf::open(in_path, in, err)) { jepa_log("jepa: cannot read GGUF '%s': %s\n", in_path, err.c_str()); return -1; }
    const int target = spec->type;

    // ---- plan -------------------------------------------------------------------------------------
    std::vector<plan_item> plan(in.tensors.size());
    std::map<int, int64_t> after_count;
    int n_fallback = 0;
    uint64_t off = 0;
    for (size_t i = 0; i < in.tensors.size(); i++) {
        plan_item & it = plan[i];
        it.t = &in.tensors[i];
        const gguf::tensor_info & t = *it.t;
        it.n_dims = 4;
        while (it.n_dims > 1 && t.ne[it.n_dims - 1] == 1) it.n_dims--;
        int dst = t.type;
        if (target == T_F32) {
            dst = T_F32;
            if (t.type != T_F32) it.note = is_quantized(t.type) ? "dequantized" : "widened";
        } else if (!is_quantizable(t.name, it.n_dims)) {
            it.note = "kept (rule)";
        } else if (std::any_of(keep, keep + std::max(n_keep, 0), [&](const char * k) { return k && t.name.find(k) != std::string::npos; })) {
            it.note = "kept (keep list)";
        } else {
            dst = target;
            if (is_quantized(t.type) && t.type != target && is_quantized(target)) {
                if (!allow_requant) {
                    jepa_log("jepa: %s is already %s; re-quantizing to %s needs allow_requant\n", t.name.c_str(), ggml_traits(t.type).name,
                             spec->name);
                    return -1;
                }
                it.note = std::string("re-quantized from ") + ggml_traits(t.type).name;
            }
            if (dst == T_Q4_K && t.ne[0] % 256 != 0) {
                it.note = "fallback q4_K -> q4_0 (ne[0]=" + std::to_string(t.ne[0]) + " not a multiple of 256)";
                dst = T_Q4_0;
                n_fallback++;
            }
            if (t.ne[0] % ggml_traits(dst).blck != 0) {
                it.note = "kept: ne[0]=" + std::to_string(t.ne[0]) + " not a multiple of the " + ggml_traits(dst).name + " block size";
                dst = t.type;
            }
            if (is_quantized(t.type) && !is_quantized(dst) && dst != t.type) it.note = "dequantized";
        }
        if (dst != t.type && !(t.type == T_F32 || t.type == T_F16 || t.type == T_BF16 || t.type == T_Q8_0 || t.type == T_Q4_0 ||
                               t.type == T_Q4_K)) {
            jepa_log("jepa: cannot convert %s from %s\n", t.name.c_str(), ggml_traits(t.type).name);
            return -1;
        }
        it.dst = dst;
        const int64_t rows = t.ne[1] * t.ne[2] * t.ne[3];
        it.dst_bytes = (uint64_t) (t.ne[0] / ggml_traits(dst).blck * ggml_traits(dst).bytes) * (uint64_t) rows;
        it.dst_offset = off;
        off += pad32(it.dst_bytes);
        if (is_quantized(dst)) after_count[dst]++;
        if (verbose && dst != t.type)
            jepa_log("jepa-quantize: %-40s %5s -> %-5s %s\n", t.name.c_str(), ggml_traits(t.type).name, ggml_traits(dst).name, it.note.c_str());
    }
    // file type: the target's, or the majority quantized type after fallbacks (moved to the end)
    uint32_t ftype = spec->ftype;
    bool ftype_to_end = false;
    if (n_fallback > 0 && is_quantized(target)) {
        int major = target;
        int64_t major_n = -1;
        for (const auto & kv : after_count) if (kv.second > major_n) { major = kv.first; major_n = kv.second; }
        if (major != target)
            for (const auto & ts : TARGETS) if (ts.type == major) { ftype = ts.ftype; ftype_to_end = true; }
    }

    // ---- metadata -----------------------------------------------------------------------------------
    std::unique_ptr<FILE, int (*)(FILE *)> fin(fopen(in_path, "rb"), fclose);
    if (!fin) { jepa_log("jepa: cannot reopen '%s'\n", in_path); return -1; }
    std::vector<std::vector<uint8_t>> kv_out;   // serialized pairs, in output order
    bool have_ft = false;
    auto ft_pair = [&]() {
        std::vector<uint8_t> b;
        const std::string key = "general.file_type";
        const uint64_t n = key.size();
        const uint32_t ty = gguf::U32;
        b.insert(b.end(), (const uint8_t *) &n, (const uint8_t *) &n + 8);
        b.insert(b.end(), key.begin(), key.end());
        b.insert(b.end(), (const uint8_t *) &ty, (const uint8_t *) &ty + 4);
        b.insert(b.end(), (const uint8_t *) &ftype, (const uint8_t *) &ftype + 4);
        return b;
    };
    for (size_t i = 0; i < in.kv.size(); i++) {
        const std::string & key = in.kv[i].first;
        if (key == "general.file_type") {
            have_ft = true;
            if (!ftype_to_end) kv_out.push_back(ft_pair());
            continue;
        }
        if (key == "general.alignment") {
            if (verbose) jepa_log("jepa-quantize: dropping general.alignment, the output uses the default alignment 32\n");
            continue;
        }
        const uint64_t b = in.kv_span[i].first, e = in.kv_span[i].second;
        std::vector<uint8_t> raw((size_t) (e - b));
        if (fseeko(fin.get(), (off_t) b, SEEK_SET) != 0 || fread(raw.data(), 1, raw.size(), fin.get()) != raw.size()) {
            jepa_log("jepa: short read of the metadata of '%s'\n", in_path);
            return -1;
        }
        kv_out.push_back(std::move(raw));
    }
    if (!have_ft || ftype_to_end) kv_out.push_back(ft_pair());

    // ---- write (a file left half-written by a failure is removed) ------------------------------------
    const int dev = device < 0 ? 0 : device;
    int prev = 0;
    hipGetDevice(&prev);
    struct restore { int d; ~restore() { hipSetDevice(d); } } rs{prev};
    if (hipSetDevice(dev) != hipSuccess) { jepa_log("jepa: jepa_amd_quantize_file: no HIP device %d\n", dev); return -1; }
    std::unique_ptr<FILE, int (*)(FILE *)> fout(fopen(out_path, "wb"), fclose);
    if (!fout) { jepa_log("jepa: cannot write '%s'\n", out_path); return -1; }
    struct remove_on_failure {
        const char * path;
        bool keep = false;
        ~remove_on_failure() { if (!keep) remove(path); }
    } guard{out_path};
    writer w{fout.get()};
    w.bytes("GGUF", 4);
    w.put<uint32_t>(3);
    w.put<uint64_t>(in.tensors.size());
    w.put<uint64_t>(kv_out.size());
    uint64_t pos = 24;
    for (const auto & b : kv_out) { w.bytes(b.data(), b.size()); pos += b.size(); }
    for (const plan_item & it : plan) {
        w.str(it.t->name);
        w.put<uint32_t>((uint32_t) it.n_dims);
        for (int d = 0; d < it.n_dims; d++) w.put<int64_t>(it.t->ne[d]);
        w.put<uint32_t>((uint32_t) it.dst);
        w.put<uint64_t>(it.dst_offset);
        pos += 8 + it.t->name.size() + 4 + 8 * (uint64_t) it.n_dims + 4 + 8;
    }
    w.zeros((size_t) (pad32(pos) - pos));

    // ---- data: unchanged tensors copied, the others through f32 on the GPU ----------------------------
    dev_buf d_src, d_f32, d_dst;
    std::vector<uint8_t> src, dst;
    int n_changed = 0;
    for (const plan_item & it : plan) {
        const gguf::tensor_info & t = *it.t;
        src.resize((size_t) t.nbytes);
        if (fseeko(fin.get(), (off_t) t.offset, SEEK_SET) != 0 || fread(src.data(), 1, src.size(), fin.get()) != src.size()) {
            jepa_log("jepa: short read on %s\n", t.name.c_str());
            return -1;
        }
        if (it.dst == t.type) {
            w.bytes(src.data(), src.size());
        } else {
            const int64_t n = t.ne[0] * t.ne[1] * t.ne[2] * t.ne[3];
            if (!d_src.need(src.size()) || !d_f32.need((size_t) n * 4) || !d_dst.need((size_t) it.dst_bytes)) {
                jepa_log("jepa: jepa_amd_quantize_file: device allocation for %s failed\n", t.name.c_str());
                return -1;
            }
            bool ok = hipMemcpy(d_src.p, src.data(), src.size(), hipMemcpyHostToDevice) == hipSuccess;
            if (ok) launch_dequant_rows(t.type, d_src.p, t.ne[1] * t.ne[2] * t.ne[3], t.ne[0], (float *) d_f32.p, nullptr);
            if (ok && it.dst != T_F32) ok = launch_quantize_rows(it.dst, (const float *) d_f32.p, n, d_dst.p, nullptr);
            dst.resize((size_t) it.dst_bytes);
            ok = ok && hipMemcpy(dst.data(), it.dst == T_F32 ? d_f32.p : d_dst.p, dst.size(), hipMemcpyDeviceToHost) == hipSuccess;
            if (!ok) { jepa_log("jepa: quantizing %s failed on the device\n", t.name.c_str()); return -1; }
            w.bytes(dst.data(), dst.size());
            n_changed++;
        }
        w.zeros((size_t) (pad32(it.dst_bytes) - it.dst_bytes));
    }
    if (!w.ok || fflush(fout.get()) != 0) { jepa_log("jepa: write error on '%s'\n", out_path); return -1; }
    if (verbose)
        jepa_log("jepa-quantize: %s -> %s [%s]: %d tensors re-typed, %d K-quant fallbacks, general.file_type %u\n", in_path, out_path,
                 spec->name, n_changed, n_fallback, ftype);
    guard.keep = true;
    return 0;
}
