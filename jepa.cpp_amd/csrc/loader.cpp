// loader.cpp - GGUF -> hparams -> validated weights on one HIP device.
//
// Follows reference src/jepa-gguf.cpp: the same jepa.* keys and defaults (254-596), the same range
// refusals by key name (240-250), the file-extent check before any allocation (821-854), the same
// tensor presence / shape / dtype rules (631-728, 942-1092). Differences: the tensors go to a HIP
// device and the matmul weights are expanded into the GEMM kernel's operand layout (dev_linear).
#include "model.h"
#include "kernels.h"

#include <algorithm>
#include <cinttypes>
#include <cmath>
#include <cstdarg>
#include <cstdio>
#include <cstring>
#include <memory>

const char * jepa_file_type_name_u32(uint32_t ft) {
    switch ((int32_t) ft) {   // GGML_FTYPE_* numbering (reference src/jepa-gguf.cpp:62-93)
        case 0: return "f32";   case 1: return "f16";   case 2: return "q4_0"; case 3: return "q4_1";
        case 4: return "q4_1_some_f16"; case 7: return "q8_0"; case 8: return "q5_0"; case 9: return "q5_1";
        case 10: return "q2_k"; case 11: return "q3_k"; case 12: return "q4_k"; case 13: return "q5_k";
        case 14: return "q6_k"; case 24: return "bf16";
        default: return "unknown";
    }
}

family_id family_from_string(const std::string & s) {
    if (s == "ijepa") return FAM_IJEPA;
    if (s == "vjepa") return FAM_VJEPA;
    if (s == "vjepa2") return FAM_VJEPA2;
    if (s == "vjepa2_1") return FAM_VJEPA2_1;
    if (s == "levjepa") return FAM_LEVJEPA;
    if (s == "hfvit") return FAM_HFVIT;
    if (s == "lewm") return FAM_LEWM;
    if (s == "hjepa") return FAM_HJEPA;
    return FAM_UNKNOWN;
}

namespace {

struct kv {
    const gguf::file & f;
    bool has(const char * k) const { return f.find(k) != nullptr; }
    int64_t geti(const char * k, int64_t def) const {
        const gguf::value * v = f.find(k);
        if (!v || v->type == gguf::STR || v->type == gguf::ARR) return def;
        return v->i;
    }
    bool getb(const char * k, bool def) const { return geti(k, def ? 1 : 0) != 0; }
    float getf(const char * k, float def) const {
        const gguf::value * v = f.find(k);
        if (!v || v->type == gguf::STR || v->type == gguf::ARR) return def;
        return (float) v->f;
    }
    std::string gets(const char * k, const std::string & def) const {
        const gguf::value * v = f.find(k);
        return v && v->type == gguf::STR ? v->s : def;
    }
    bool farr(const char * k, float * out, size_t n) const {
        const gguf::value * v = f.find(k);
        if (!v || v->type != gguf::ARR || v->arr_type == gguf::STR || v->af.size() != n) return false;
        for (size_t i = 0; i < n; i++) out[i] = (float) v->af[i];
        return true;
    }
};

bool kv_range(const char * key, int64_t v, int64_t lo, int64_t hi) {
    if (v >= lo && v <= hi) return true;
    jepa_log("jepa: %s = %" PRId64 " is out of range [%" PRId64 ", %" PRId64 "]\n", key, v, lo, hi);
    return false;
}

bool kv_finite(const char * key, float v, float lo, float hi) {
    if (v >= lo && v <= hi) return true;
    jepa_log("jepa: %s = %g is not a finite value in [%g, %g]\n", key, (double) v, (double) lo, (double) hi);
    return false;
}

bool act_from_string(const std::string & s, act_id & a) {
    if (s == "gelu_erf" || s == "gelu") { a = ACT_GELU_ERF; return true; }
    if (s == "gelu_tanh" || s == "gelu_new" || s == "gelu_pytorch_tanh") { a = ACT_GELU_TANH; return true; }
    if (s == "silu" || s == "swish") { a = ACT_SILU; return true; }
    if (s == "relu") { a = ACT_RELU; return true; }
    jepa_log("jepa: unknown activation '%s' (expected gelu_erf | gelu_tanh | silu | relu)\n", s.c_str());
    return false;
}

bool hparams_from_gguf(const gguf::file & f, hparams & hp, std::vector<std::pair<std::string, std::string>> & raw) {
    kv r{f};
    for (const auto & p : f.kv)
        if (p.first.rfind("general.", 0) == 0 || p.first.rfind("jepa.", 0) == 0) raw.emplace_back(p.first, p.second.render());
    hp.arch = r.gets("general.architecture", "");
    hp.name = r.gets("general.name", "");
    hp.file_type = (uint32_t) r.geti("general.file_type", 0);
    if (hp.arch != "jepa") { jepa_log("jepa: general.architecture is '%s', expected 'jepa'\n", hp.arch.c_str()); return false; }
    hp.family_str = r.gets("jepa.family", "");
    hp.family = family_from_string(hp.family_str);
    hp.modality = r.gets("jepa.modality", "image");
    if (hp.family == FAM_UNKNOWN) { jepa_log("jepa: unknown jepa.family '%s'\n", hp.family_str.c_str()); return false; }

    enc_hparams & e = hp.enc;
    for (const char * k : {"jepa.enc.embed_dim", "jepa.enc.n_layer", "jepa.enc.n_head", "jepa.enc.ffn_dim", "jepa.enc.patch_size"})
        if (!r.has(k)) { jepa_log("jepa: missing required key %s\n", k); return false; }
    const int64_t ed = r.geti("jepa.enc.embed_dim", 0), nl = r.geti("jepa.enc.n_layer", 0), nh = r.geti("jepa.enc.n_head", 0);
    const int64_t ff = r.geti("jepa.enc.ffn_dim", 0), ps = r.geti("jepa.enc.patch_size", 16), tb = r.geti("jepa.enc.tubelet_size", 1);
    const int64_t is = r.geti("jepa.enc.img_size", 224), nf = r.geti("jepa.enc.n_frames", 1), ic = r.geti("jepa.enc.in_chans", 3);
    if (!kv_range("jepa.enc.embed_dim", ed, 1, JEPA_LIMIT_EMBED_DIM) || !kv_range("jepa.enc.n_layer", nl, 1, JEPA_LIMIT_N_LAYER) ||
        !kv_range("jepa.enc.n_head", nh, 1, JEPA_LIMIT_N_HEAD) || !kv_range("jepa.enc.ffn_dim", ff, 1, JEPA_LIMIT_FFN_DIM) ||
        !kv_range("jepa.enc.patch_size", ps, 1, JEPA_LIMIT_PATCH_SIZE) || !kv_range("jepa.enc.tubelet_size", tb, 1, JEPA_LIMIT_PATCH_SIZE) ||
        !kv_range("jepa.enc.img_size", is, 1, JEPA_LIMIT_IMG_SIZE) || !kv_range("jepa.enc.n_frames", nf, 1, JEPA_LIMIT_N_FRAMES) ||
        !kv_range("jepa.enc.in_chans", ic, 1, JEPA_LIMIT_IN_CHANS)) return false;
    e.embed_dim = (int) ed; e.n_layer = (int) nl; e.n_head = (int) nh; e.ffn_dim = (int) ff; e.patch_size = (int) ps;
    e.tubelet_size = (int) tb; e.img_size = (int) is; e.n_frames = (int) nf; e.in_chans = (int) ic;
    e.ln_eps = r.getf("jepa.enc.ln_eps", 1e-6f);
    if (!kv_finite("jepa.enc.ln_eps", e.ln_eps, 0.0f, 1.0f)) return false;
    if (!act_from_string(r.gets("jepa.enc.act", "gelu_erf"), e.act)) return false;
    e.pos_type = r.gets("jepa.enc.pos_type", "");
    e.rope_theta = r.getf("jepa.enc.rope_theta", 10000.0f);
    e.rope_interpolate = r.getb("jepa.enc.rope_interpolate", false);
    e.rope_freq_layout = r.gets("jepa.enc.rope_freq_layout", "");
    e.rope_ref_grid = (int) r.geti("jepa.enc.rope_ref_grid", 0);
    e.cls_token = r.getb("jepa.enc.cls_token", false);
    const int64_t nreg = r.geti("jepa.enc.n_registers", 0);
    e.qkv_fused = r.getb("jepa.enc.qkv_fused", true);
    e.modality_embed = r.getb("jepa.enc.modality_embed", false);
    e.image_patch_embed = r.getb("jepa.enc.image_patch_embed", false);
    e.layer_scale = r.getb("jepa.enc.layer_scale", false);
    e.attn_mode = r.gets("jepa.enc.attn_mode", "full");
    if (e.attn_mode != "full" && e.attn_mode != "block_causal") {
        jepa_log("jepa: unknown jepa.enc.attn_mode '%s' (expected full | block_causal)\n", e.attn_mode.c_str());
        return false;
    }
    // only the video encoder graph builds the mask; an image family would run unmasked, which is
    // what the key exists to prevent (reference tests/test-errors.cpp:259-262)
    if (e.attn_mode == "block_causal" && !is_video_family(hp.family)) {
        jepa_log("jepa: jepa.enc.attn_mode 'block_causal' is only defined for the video families (family '%s')\n",
                 hp.family_str.c_str());
        return false;
    }
    e.has_proj = r.has("jepa.enc.proj_act");
    if (!kv_range("jepa.enc.n_registers", nreg, 0, JEPA_LIMIT_N_TOKENS)) return false;
    e.n_registers = (int) nreg;
    if (!kv_finite("jepa.enc.rope_theta", e.rope_theta, 1e-6f, 1e12f)) return false;
    if (!kv_range("jepa.enc.rope_ref_grid", e.rope_ref_grid, 0, JEPA_LIMIT_IMG_SIZE)) return false;
    if (e.rope_interpolate && e.rope_ref_grid < 1) {
        jepa_log("jepa: jepa.enc.rope_interpolate is set but jepa.enc.rope_ref_grid is %d - interpolation has no training grid to rescale from\n",
                 e.rope_ref_grid);
        return false;
    }
    if (e.embed_dim % e.n_head != 0) { jepa_log("jepa: embed_dim %d not divisible by n_head %d\n", e.embed_dim, e.n_head); return false; }
    const bool rope = is_video_family(hp.family) || hp.family == FAM_LEVJEPA || e.pos_type == "rope3d";
    if (rope && e.head_dim() % 2 != 0) {
        jepa_log("jepa: 3-D RoPE rotates pairs, so the encoder head width has to be even; embed_dim %d / n_head %d is %d\n",
                 e.embed_dim, e.n_head, e.head_dim());
        return false;
    }
    hp.has_pred = r.has("jepa.pred.kind") && r.gets("jepa.pred.kind", "none") != "none";
    hp.pred_kind = r.gets("jepa.pred.kind", "");
    if (hp.has_pred) {
        // src/jepa-gguf.cpp:379-440
        pred_hparams & p = hp.pred;
        p.kind = hp.pred_kind;
        const int64_t ped = r.geti("jepa.pred.embed_dim", 0), pnl = r.geti("jepa.pred.n_layer", 0), pnh = r.geti("jepa.pred.n_head", 0);
        const int64_t pff = r.geti("jepa.pred.ffn_dim", 0), phd = r.geti("jepa.pred.head_dim", 0), pnm = r.geti("jepa.pred.n_mask_tokens", 0);
        const int64_t pod = r.geti("jepa.pred.out_dim", e.embed_dim), pgs = r.geti("jepa.pred.grid_size", 0);
        const int64_t prg = r.geti("jepa.pred.rope_ref_grid", 0);
        if (!kv_range("jepa.pred.embed_dim", ped, 1, JEPA_LIMIT_EMBED_DIM) || !kv_range("jepa.pred.n_layer", pnl, 1, JEPA_LIMIT_N_LAYER) ||
            !kv_range("jepa.pred.n_head", pnh, 1, JEPA_LIMIT_N_HEAD) || !kv_range("jepa.pred.ffn_dim", pff, 1, JEPA_LIMIT_FFN_DIM) ||
            !kv_range("jepa.pred.out_dim", pod, 1, JEPA_LIMIT_FFN_DIM) || !kv_range("jepa.pred.head_dim", phd, 0, JEPA_LIMIT_EMBED_DIM) ||
            !kv_range("jepa.pred.n_mask_tokens", pnm, 0, JEPA_LIMIT_N_TOKENS) ||
            !kv_range("jepa.pred.grid_size", pgs, 0, JEPA_LIMIT_IMG_SIZE) || !kv_range("jepa.pred.rope_ref_grid", prg, 0, JEPA_LIMIT_IMG_SIZE))
            return false;
        p.embed_dim = (int) ped; p.n_layer = (int) pnl; p.n_head = (int) pnh; p.ffn_dim = (int) pff; p.head_dim = (int) phd;
        p.n_mask_tokens = (int) pnm; p.out_dim = (int) pod; p.grid_size = (int) pgs; p.rope_ref_grid = (int) prg;
        p.rope_freq_layout = r.gets("jepa.pred.rope_freq_layout", "");
        p.rope_interpolate = r.getb("jepa.pred.rope_interpolate", false);
        p.modality_embed = r.getb("jepa.pred.modality_embed", false);
        if (!act_from_string(r.gets("jepa.pred.act", "gelu_erf"), p.act)) return false;
        if (p.head_dim == 0 && p.embed_dim % p.n_head != 0) {
            jepa_log("jepa: jepa.pred.embed_dim %d is not divisible by jepa.pred.n_head %d and there is no jepa.pred.head_dim\n",
                     p.embed_dim, p.n_head);
            return false;
        }
        if (p.rope_interpolate && p.rope_ref_grid <= 0) {
            jepa_log("jepa: jepa.pred.rope_interpolate is set but jepa.pred.rope_ref_grid is %d\n", p.rope_ref_grid);
            return false;
        }
    }
    hp.head_kind = r.gets("jepa.head.kind", "none");
    hp.has_head = hp.head_kind != "none" && !hp.head_kind.empty();
    if (hp.has_head) {
        hp.n_classes = (int) r.geti("jepa.head.n_classes", 0);
        const gguf::value * lv = f.find("jepa.head.labels");
        if (lv && lv->type == gguf::ARR && lv->arr_type == gguf::STR) hp.labels = lv->as;
        hp.n_pool_layers = (int) r.geti("jepa.head.n_pool_layers", 0);
        if (!kv_range("jepa.head.n_classes", hp.n_classes, 0, JEPA_LIMIT_N_TOKENS) ||
            !kv_range("jepa.head.n_pool_layers", hp.n_pool_layers, 0, JEPA_LIMIT_N_LAYER) ||
            !kv_range("jepa.head.labels length", (int64_t) hp.labels.size(), 0, JEPA_LIMIT_N_TOKENS)) return false;
    }
    pre_hparams & pre = hp.pre;
    r.farr("jepa.pre.mean", pre.mean, 3);
    r.farr("jepa.pre.std", pre.std, 3);
    pre.resize_short = (int) r.geti("jepa.pre.resize_short", e.img_size);
    pre.crop = (int) r.geti("jepa.pre.crop", e.img_size);
    pre.resample = r.gets("jepa.pre.resample", "bilinear");
    pre.resize_mode = r.gets("jepa.pre.resize_mode", "shortest_edge");
    pre.rescale = r.getf("jepa.pre.rescale", 1.0f / 255.0f);
    if (!kv_range("jepa.pre.resize_short", pre.resize_short, 1, JEPA_LIMIT_IMG_SIZE) ||
        !kv_range("jepa.pre.crop", pre.crop, 0, JEPA_LIMIT_IMG_SIZE) || !kv_finite("jepa.pre.rescale", pre.rescale, 1e-9f, 1e9f))
        return false;
    for (int i = 0; i < 3; i++) {
        if (!kv_finite("jepa.pre.mean", pre.mean[i], -1e6f, 1e6f)) return false;
        if (!kv_finite("jepa.pre.std", pre.std[i], 1e-9f, 1e6f)) return false;
    }
    return true;
}

struct loader {
    jepa_model * m;
    const gguf::file & f;
    FILE * fp;
    hipStream_t s;
    void * staging = nullptr;
    size_t staging_size = 0;
    std::vector<uint8_t> host;

    void * dalloc(size_t bytes) {
        void * p = nullptr;
        if (bytes == 0) bytes = 16;
        if (hipMalloc(&p, bytes) != hipSuccess) {
            jepa_log("jepa: hipMalloc of %.1f MiB failed on device %d\n", bytes / 1048576.0, m->device);
            return nullptr;
        }
        m->allocations.push_back(p);
        m->n_bytes_weights += bytes;
        return p;
    }

    bool read(const gguf::tensor_info & t) {
        host.resize(t.nbytes);
        if (fseeko(fp, (off_t) t.offset, SEEK_SET) != 0 || fread(host.data(), 1, t.nbytes, fp) != t.nbytes) {
            jepa_log("jepa: short read for tensor %s (%" PRIu64 " bytes @ %" PRIu64 ")\n", t.name.c_str(), t.nbytes, t.offset);
            return false;
        }
        m->n_bytes_file += t.nbytes;
        return true;
    }

    // the tensor's bytes into device staging, followed by pad_bytes of zeros (zero rows: d = 0 in
    // every quantized block format, so they dequantize to 0)
    bool to_staging(const gguf::tensor_info & t, size_t pad_bytes = 0) {
        if (!read(t)) return false;
        const size_t need = t.nbytes + pad_bytes;
        if (staging_size < need) {
            if (staging) hipFree(staging);
            staging = nullptr;
            staging_size = 0;
            if (hipMalloc(&staging, need) != hipSuccess) { jepa_log("jepa: hipMalloc(staging) failed\n"); return false; }
            staging_size = need;
        }
        return hipMemcpyAsync(staging, host.data(), t.nbytes, hipMemcpyHostToDevice, s) == hipSuccess &&
               (pad_bytes == 0 || hipMemsetAsync((char *) staging + t.nbytes, 0, pad_bytes, s) == hipSuccess) &&
               hipStreamSynchronize(s) == hipSuccess;
    }

    // an f32 vector of exactly n values (norms, biases, tokens, tables) - src/jepa-gguf.cpp:675-701
    // (n_alloc > n: the device copy is n_alloc values, the tail zero)
    bool vec(const std::string & name, int64_t n, float ** out, bool required = false, int64_t n_alloc = 0) {
        const gguf::tensor_info * t = f.tensor(name);
        if (!t) {
            if (required) { jepa_log("jepa: required tensor '%s' missing from %s\n", name.c_str(), m->path.c_str()); return false; }
            return true;
        }
        if (t->type != T_F32) {
            jepa_log("jepa: tensor %s is %s, but it is added to or concatenated with the f32 activations and has to be f32 "
                     "(only the matmul weights may be quantized)\n", name.c_str(), ggml_traits(t->type).name);
            return false;
        }
        int64_t nel = t->ne[0] * t->ne[1] * t->ne[2] * t->ne[3];
        if (n >= 0 && nel != n) {
            jepa_log("jepa: tensor %s holds %" PRId64 " values, expected %" PRId64 "\n", name.c_str(), nel, n);
            return false;
        }
        if (!read(*t)) return false;
        const size_t bytes = std::max<size_t>(t->nbytes, (size_t) n_alloc * 4);
        float * d = (float *) dalloc(bytes);
        if (!d || (bytes > t->nbytes && hipMemset(d, 0, bytes) != hipSuccess) ||
            hipMemcpy(d, host.data(), t->nbytes, hipMemcpyHostToDevice) != hipSuccess) return false;
        *out = d;
        return true;
    }

    // rows (ne[1]) of a 2-D tensor, 0 when it is absent
    int64_t rows_of(const std::string & name) const {
        const gguf::tensor_info * t = f.tensor(name);
        return t ? t->ne[1] : 0;
    }

    // several tensors into device staging back to back, then pad_bytes of zeros
    bool to_staging_n(const std::vector<const gguf::tensor_info *> & ts, size_t pad_bytes) {
        if (ts.size() == 1) return to_staging(*ts[0], pad_bytes);
        size_t total = pad_bytes;
        for (const auto * t : ts) total += t->nbytes;
        if (staging_size < total) {
            if (staging) hipFree(staging);
            staging = nullptr;
            staging_size = 0;
            if (hipMalloc(&staging, total) != hipSuccess) { jepa_log("jepa: hipMalloc(staging) failed\n"); return false; }
            staging_size = total;
        }
        size_t off = 0;
        for (const auto * t : ts) {   // host buffer reused per tensor: each copy completes before the next read
            if (!read(*t) || hipMemcpyAsync((char *) staging + off, host.data(), t->nbytes, hipMemcpyHostToDevice, s) != hipSuccess ||
                hipStreamSynchronize(s) != hipSuccess) return false;
            off += t->nbytes;
        }
        return pad_bytes == 0 || (hipMemsetAsync((char *) staging + off, 0, pad_bytes, s) == hipSuccess && hipStreamSynchronize(s) == hipSuccess);
    }

    // pad_out: the device matrix gets n_out rounded up to 128 rows (zero weights and bias), for the
    // linears whose output count the file chooses freely (the classifier); L.n_valid keeps n_out
    bool linear(const std::string & wname, const std::string & bname, int64_t n_in, int64_t n_out, dev_linear & L, bool required,
                bool pad_out = false) {
        return linear_n({wname}, {bname}, n_in, n_out, L, required, pad_out);
    }

    // One device linear from the weight tensors wnames stacked along the outputs (each [n_in, n_out /
    // parts], the same dtype; quantized blocks never cross a row, so the stacked rows are the fused
    // matrix's) with their biases likewise: the separate attn_q / attn_k / attn_v of an unfused block,
    // whose three linears the reference runs one by one (src/jepa.cpp:408-414)
    bool linear_n(const std::vector<std::string> & wnames, const std::vector<std::string> & bnames, int64_t n_in, int64_t n_out,
                  dev_linear & L, bool required, bool pad_out = false) {
        const std::string & wname = wnames[0];
        const int64_t n_part = n_out / (int64_t) wnames.size();
        std::vector<const gguf::tensor_info *> ts;
        for (const auto & name : wnames) {
            const gguf::tensor_info * t = f.tensor(name);
            if (!t) {
                if (required || !ts.empty()) { jepa_log("jepa: required tensor '%s' missing from %s\n", name.c_str(), m->path.c_str()); return false; }
                return true;
            }
            if (t->ne[0] != n_in || t->ne[1] != n_part || t->ne[2] != 1 || t->ne[3] != 1) {
                jepa_log("jepa: tensor %s has shape [%" PRId64 ", %" PRId64 "], expected [%" PRId64 ", %" PRId64 "]\n",
                         name.c_str(), t->ne[0], t->ne[1], n_in, n_part);
                return false;
            }
            ts.push_back(t);
        }
        // Parts of different dtypes: the reference runs each part as its own linear. q8_0 and q4_0 parts
        // mix exactly: both take q8_0 activations and q4_0's codes q - 8 are int8 codes under the same
        // f16 scale, so every part expands to the int8 layout and one GEMM gives each part's own dot
        // products. Any other mix needs different activation formats per part: block() loads those
        // parts as separate linears and never stacks them here.
        bool mixed = false;
        for (const auto * p : ts) mixed |= p->type != ts[0]->type;
        if (mixed) {
            for (const auto * p : ts)
                if (p->type != T_Q8_0 && p->type != T_Q4_0) {
                    jepa_log("jepa: the parts of %s are of different dtypes (%s, ...): only q8_0 and q4_0 parts can be "
                             "mixed in one linear here\n", wname.c_str(), ggml_traits(p->type).name);
                    return false;
                }
        }
        const gguf::tensor_info * t = ts[0];
        size_t nbytes = 0;
        for (const auto * p : ts) nbytes += p->nbytes;
        const int64_t n_file = n_out;
        if (pad_out) n_out = (n_out + 127) / 128 * 128;
        const size_t pad_bytes = (size_t) (n_out - n_file) * (nbytes / (size_t) n_file);
        L.gtype = mixed ? (int) T_Q8_0 : t->type; L.n_in = n_in; L.n_out = n_out; L.n_valid = n_file;
        L.fmt = mixed ? (int) W_Q32 : weight_format(t->type, n_in);
        if (L.fmt < 0) {
            jepa_log("jepa: tensor %s has dtype %s, which this engine has no GEMM kernel for "
                     "(f32, f16, q8_0, q4_0 and q4_K are supported)\n", wname.c_str(), ggml_traits(t->type).name);
            return false;
        }
        if (L.fmt != W_F32 && (n_out % 128 != 0 || n_in % 64 != 0)) {
            jepa_log("jepa: tensor %s is [%" PRId64 " x %" PRId64 "]: the MFMA GEMM needs rows that are a multiple of 64 and a "
                     "multiple of 128 outputs\n", wname.c_str(), n_in, n_out);
            return false;
        }
        if (L.fmt == W_F32 && n_out % 4 != 0) {
            jepa_log("jepa: tensor %s: %" PRId64 " outputs is not a multiple of 4\n", wname.c_str(), n_out);
            return false;
        }
        if (!to_staging_n(ts, pad_bytes)) return false;
        if (L.fmt == W_F32 || L.fmt == W_F16) {
            L.w = dalloc(nbytes + pad_bytes);
            if (!L.w || hipMemcpyAsync(L.w, staging, nbytes + pad_bytes, hipMemcpyDeviceToDevice, s) != hipSuccess) return false;
        } else {
            L.w = dalloc(weight_code_bytes(L.fmt, n_out, n_in));
            if (!L.w) return false;
            if (L.fmt == W_Q32 || L.fmt == W_Q40) {
                L.wd = dalloc((size_t) n_out * (n_in / 32) * 2);
                if (!L.wd) return false;
            } else {
                L.wd = dalloc((size_t) n_out * (n_in / 256) * 4);
                L.wmin = dalloc((size_t) n_out * (n_in / 256) * 16 * 2);
                if (!L.wd || !L.wmin) return false;
            }
            if (!mixed) {
                launch_repack(t->type, staging, n_out, n_in, L.w, L.wd, L.wmin, s);
            } else {
                size_t off = 0;
                for (size_t p = 0; p < ts.size(); p++) {
                    launch_repack(ts[p]->type, (const char *) staging + off, n_part, n_in, (int8_t *) L.w + (size_t) p * n_part * n_in,
                                  (uint16_t *) L.wd + (size_t) p * n_part * (n_in / 32), nullptr, s, true);
                    off += ts[p]->nbytes;
                }
            }
        }
        if (hipStreamSynchronize(s) != hipSuccess) { jepa_log("jepa: weight upload of %s failed\n", wname.c_str()); return false; }
        if (bnames.size() == 1) return vec(bnames[0], n_file, &L.bias, false, n_out);
        // stacked biases, each optional on its own (the reference adds each part's bias when present,
        // src/jepa.cpp:408-414, src/jepa-gguf.cpp:712-714): an absent part adds zeros
        int present = 0;
        for (const auto & b : bnames) present += f.tensor(b) ? 1 : 0;
        if (present == 0) return true;
        std::vector<float> all;
        for (const auto & b : bnames) {
            const gguf::tensor_info * bt = f.tensor(b);
            if (!bt) {
                all.insert(all.end(), (size_t) n_part, 0.0f);
                continue;
            }
            if (bt->type != T_F32 || bt->ne[0] * bt->ne[1] * bt->ne[2] * bt->ne[3] != n_part) {
                jepa_log("jepa: bias %s has to be f32 with %" PRId64 " values\n", b.c_str(), n_part);
                return false;
            }
            if (!read(*bt)) return false;
            const float * v = (const float *) host.data();
            all.insert(all.end(), v, v + n_part);
        }
        all.resize((size_t) n_out, 0.0f);
        L.bias = (float *) dalloc(all.size() * 4);
        return L.bias && hipMemcpy(L.bias, all.data(), all.size() * 4, hipMemcpyHostToDevice) == hipSuccess;
    }

    // one pre-LN block "<p>ln1.weight" ... (src/jepa-gguf.cpp:236-252 names) of FFN width F (0: the
    // ffn_up tensor's row count)
    bool block(const std::string & p, int64_t D, int64_t F, dev_layer & Ly, int64_t inner = 0) {
        if (inner <= 0) inner = D;   // attention width n_head * head_dim
        // the attention input projection: attn_qkv, or attn_q / attn_k / attn_v (the reference uses
        // attn_qkv when the file has it, src/jepa.cpp:399-414)
        const bool fused = f.tensor(p + "attn_qkv.weight") != nullptr;
        const bool split = f.tensor(p + "attn_q.weight") && f.tensor(p + "attn_k.weight") && f.tensor(p + "attn_v.weight");
        if (!f.tensor(p + "ln1.weight") || !f.tensor(p + "ln2.weight") || !f.tensor(p + "attn_out.weight") || !f.tensor(p + "ffn_up.weight") ||
            !f.tensor(p + "ffn_down.weight") || (!fused && !split)) {
            jepa_log("jepa: block %s* is incomplete: needs ln1/ln2/attn_out/ffn_up/ffn_down and attn_qkv (or attn_q/k/v)\n", p.c_str());
            return false;
        }
        if (F <= 0) F = rows_of(p + "ffn_up.weight");
        // separate q / k / v stack into one linear when their dtypes agree or are q8_0 / q4_0 (one
        // activation format); other mixes stay three linears, each with its own activation format
        static const char * const QKV[3] = {"attn_q", "attn_k", "attn_v"};
        if (!fused) {
            bool same = true, int8_family = true;
            for (const char * q : QKV) {
                const int ty = f.tensor(p + q + ".weight")->type;
                same &= ty == f.tensor(p + "attn_q.weight")->type;
                int8_family &= ty == T_Q8_0 || ty == T_Q4_0;
            }
            Ly.qkv_separate = !same && !int8_family;
        }
        bool qkv_ok = true;
        if (fused) qkv_ok = linear(p + "attn_qkv.weight", p + "attn_qkv.bias", D, 3 * inner, Ly.qkv, true);
        else if (!Ly.qkv_separate)
            qkv_ok = linear_n({p + "attn_q.weight", p + "attn_k.weight", p + "attn_v.weight"},
                              {p + "attn_q.bias", p + "attn_k.bias", p + "attn_v.bias"}, D, 3 * inner, Ly.qkv, true);
        else
            for (int i = 0; i < 3 && qkv_ok; i++)
                qkv_ok = linear(p + QKV[i] + ".weight", p + QKV[i] + ".bias", D, inner, Ly.qkv_part[i], true);
        return qkv_ok && vec(p + "ln1.weight", D, &Ly.ln1_w) && vec(p + "ln1.bias", D, &Ly.ln1_b) && vec(p + "ln2.weight", D, &Ly.ln2_w) &&
               vec(p + "ln2.bias", D, &Ly.ln2_b) && vec(p + "ls1", D, &Ly.ls1) && vec(p + "ls2", D, &Ly.ls2) &&
               linear(p + "attn_out.weight", p + "attn_out.bias", inner, D, Ly.out, true) &&
               linear(p + "ffn_up.weight", p + "ffn_up.bias", D, F, Ly.up, true) &&
               linear(p + "ffn_down.weight", p + "ffn_down.bias", F, D, Ly.down, true);
    }
};

}  // namespace

bool is_video_family(family_id f) { return f == FAM_VJEPA2 || f == FAM_VJEPA2_1 || f == FAM_LEVJEPA; }
bool is_image_family(family_id f) { return f == FAM_IJEPA || f == FAM_HFVIT || f == FAM_LEWM || f == FAM_HJEPA; }

static void model_free_device(jepa_model * m) {
    std::lock_guard<std::recursive_mutex> lk(jepa_hip_mutex());
    int prev = 0;
    hipGetDevice(&prev);
    hipSetDevice(m->device);
    for (void * p : m->allocations) hipFree(p);
    m->allocations.clear();
    hipSetDevice(prev);
}

extern "C" void jepa_model_free(jepa_model * m) {
    if (!m) return;
    model_free_device(m);
    delete m;
}

extern "C" jepa_model_params jepa_model_default_params(void) {
    jepa_model_params p;
    p.verbose = false;
    p.device = device_from_env();
    return p;
}

extern "C" jepa_model * jepa_model_load(const char * path, bool verbose) {
    jepa_model_params p = jepa_model_default_params();
    p.verbose = verbose;
    return jepa_model_load_ex(path, &p);
}

extern "C" jepa_model * jepa_model_load_ex(const char * path, const jepa_model_params * params) {
    if (!path || !*path) { jepa_log("jepa: jepa_model_load: no path given\n"); return nullptr; }
    const jepa_model_params mp = params ? *params : jepa_model_default_params();

    // the file is parsed and its metadata checked before any device is touched, so a broken file
    // is refused by name on any machine
    gguf::file f;
    std::string err;
    if (!gguf::open(path, f, err)) { jepa_log("jepa: cannot open GGUF %s: %s\n", path, err.c_str()); return nullptr; }
    std::unique_ptr<jepa_model> m(new jepa_model());
    m->path = path;
    if (!hparams_from_gguf(f, m->hp, m->raw_kv)) return nullptr;
    const enc_hparams & e = m->hp.enc;
    // every tensor in a jepa file is a weight, bias or table: float or quantized (src/jepa-gguf.cpp:685-701)
    for (const auto & t : f.tensors) {
        if (t.type == T_F32 || t.type == T_F16 || t.type == T_BF16 || ggml_traits(t.type).blck > 1) continue;
        jepa_log("jepa: tensor %s has dtype %s, which is not a weight dtype\n", t.name.c_str(), ggml_traits(t.type).name);
        return nullptr;
    }
    if (!is_image_family(m->hp.family) && !is_video_family(m->hp.family)) {
        // the loader accepts the file; jepa_encode reports the family as not implemented on this path
        if (mp.verbose) jepa_log("jepa: family '%s' has no encoder path in this library\n", m->hp.family_str.c_str());
    }

    const int device = dev_resolve(mp.device);
    if (device < 0) return nullptr;
    m->device = device;
    std::lock_guard<std::recursive_mutex> lk(jepa_hip_mutex());
    if (hipSetDevice(device) != hipSuccess) { jepa_log("jepa: hipSetDevice(%d) failed\n", device); return nullptr; }
    std::unique_ptr<FILE, int (*)(FILE *)> fp(fopen(path, "rb"), fclose);
    if (!fp) { jepa_log("jepa: cannot reopen %s for tensor data\n", path); return nullptr; }
    hipStream_t s = nullptr;
    if (hipStreamCreate(&s) != hipSuccess) { jepa_log("jepa: hipStreamCreate failed\n"); return nullptr; }
    loader L{m.get(), f, fp.get(), s};
    bool ok = true;
    const int64_t D = e.embed_dim;
    const int64_t patch_in = (int64_t) e.in_chans * e.tubelet_size * e.patch_size * e.patch_size;
    const bool video = is_video_family(m->hp.family);
    const bool encoder = video || is_image_family(m->hp.family);
    if (!f.tensor("enc.patch_embed.weight")) { jepa_log("jepa: enc.patch_embed.weight missing\n"); ok = false; }
    if (ok && encoder) {
        ok = L.linear("enc.patch_embed.weight", "enc.patch_embed.bias", patch_in, D, m->patch, true) &&
             L.linear("enc.patch_embed_img.weight", "enc.patch_embed_img.bias", (int64_t) e.in_chans * e.patch_size * e.patch_size, D,
                      m->patch_img, false) &&
             L.vec("enc.cls_token", D, &m->cls_token) && L.vec("enc.mod_embed_img", D, &m->mod_img) &&
             L.vec("enc.mod_embed_video", D, &m->mod_video) && L.vec("enc.norm.weight", D, &m->norm_w) &&
             L.vec("enc.norm.bias", D, &m->norm_b);
        if (ok && f.tensor("enc.pos_embed")) {
            const gguf::tensor_info * t = f.tensor("enc.pos_embed");
            if (t->ne[0] != D) { jepa_log("jepa: tensor enc.pos_embed has rows of %" PRId64 ", expected %" PRId64 "\n", t->ne[0], D); ok = false; }
            else if (!kv_range("enc.pos_embed rows", t->ne[1], 1, JEPA_LIMIT_N_TOKENS)) ok = false;
            else { m->pos_rows = t->ne[1]; ok = L.vec("enc.pos_embed", -1, &m->pos_embed); }
        }
        if (ok && e.cls_token && !m->cls_token) { jepa_log("jepa: cls_token=true but enc.cls_token missing\n"); ok = false; }
        if (ok && e.n_registers > 0) {   // enc.reg_tokens [n_registers rows of D], f32 (src/jepa-gguf.cpp:959-979)
            const gguf::tensor_info * t = f.tensor("enc.reg_tokens");
            if (!t || t->ne[0] != D || t->ne[1] != e.n_registers || t->ne[2] != 1 || t->ne[3] != 1) {
                jepa_log("jepa: jepa.enc.n_registers is %d but enc.reg_tokens is %s\n", e.n_registers, t ? "a different shape" : "missing");
                ok = false;
            } else {
                ok = L.vec("enc.reg_tokens", D * e.n_registers, &m->reg_tokens, true);
            }
        }
        m->layers.resize((size_t) e.n_layer);
        for (int i = 0; i < e.n_layer && ok; i++) ok = L.block("enc.blk." + std::to_string(i) + ".", D, e.ffn_dim, m->layers[(size_t) i]);
        if (ok && e.modality_embed && video && !m->mod_video) {
            jepa_log("jepa: jepa.enc.modality_embed is set but enc.mod_embed_video is missing\n");
            ok = false;
        }
    }
    if (ok && encoder && m->hp.has_pred && m->hp.pred.kind == "masked") {
        // src/jepa-gguf.cpp:990-1066: blocks, norm, mask tokens, embed (linear or 2-layer MLP), proj
        const pred_hparams & p = m->hp.pred;
        dev_pred & pr = m->pred;
        const int64_t Dp = p.embed_dim;
        pr.blocks.resize((size_t) p.n_layer);
        for (int i = 0; i < p.n_layer && ok; i++) ok = L.block("pred.blk." + std::to_string(i) + ".", Dp, p.ffn_dim, pr.blocks[(size_t) i],
                          (int64_t) p.n_head * p.head_dim_eff());
        const gguf::tensor_info * mt = f.tensor("pred.mask_tokens");
        if (ok && (!mt || mt->ne[0] != Dp || mt->ne[1] < 1 || mt->ne[2] != 1 || mt->ne[3] != 1)) {
            jepa_log("jepa: pred.mask_tokens is missing or not [%" PRId64 ", n] f32\n", Dp);
            ok = false;
        }
        if (ok && p.n_mask_tokens > mt->ne[1]) {
            jepa_log("jepa: jepa.pred.n_mask_tokens is %d but pred.mask_tokens holds %" PRId64 " rows\n", p.n_mask_tokens, mt->ne[1]);
            ok = false;
        }
        if (ok) pr.n_mask_rows = mt->ne[1];
        ok = ok && L.vec("pred.mask_tokens", -1, &pr.mask_tokens, true) && L.vec("pred.norm.weight", Dp, &pr.norm_w, true) &&
             L.vec("pred.norm.bias", Dp, &pr.norm_b) && L.vec("pred.mod_embed_video", Dp, &pr.mod_video) &&
             L.vec("pred.mod_embed_img", Dp, &pr.mod_img) &&
             L.linear("pred.proj.weight", "pred.proj.bias", Dp, p.out_dim, pr.proj, true);
        if (ok && f.tensor("pred.embed.0.weight")) {
            const int64_t hid = L.rows_of("pred.embed.0.weight");
            ok = L.linear("pred.embed.0.weight", "pred.embed.0.bias", D, hid, pr.embed0, true) &&
                 L.linear("pred.embed.2.weight", "pred.embed.2.bias", hid, Dp, pr.embed2, true);
        } else if (ok) {
            ok = L.linear("pred.embed.weight", "pred.embed.bias", D, Dp, pr.embed, true);
        }
    }
    if (ok && encoder && m->hp.head_kind == "attentive_pool") {
        // src/jepa-gguf.cpp:1070-1090: every head tensor is required, shapes checked against D
        dev_head & h = m->head;
        h.blocks.resize((size_t) m->hp.n_pool_layers);
        for (int i = 0; i < m->hp.n_pool_layers && ok; i++) ok = L.block("head.blk." + std::to_string(i) + ".", D, 0, h.blocks[(size_t) i]);
        const int64_t Fx = L.rows_of("head.xattn.ffn_up.weight"), C = L.rows_of("head.cls.weight");
        ok = ok && L.vec("head.query", D, &h.query, true) && L.vec("head.xattn.ln_kv.weight", D, &h.ln_kv_w, true) &&
             L.vec("head.xattn.ln_kv.bias", D, &h.ln_kv_b, true) && L.vec("head.xattn.ln2.weight", D, &h.ln2_w, true) &&
             L.vec("head.xattn.ln2.bias", D, &h.ln2_b, true) &&
             L.linear("head.xattn.q.weight", "head.xattn.q.bias", D, D, h.q, true) &&
             L.linear("head.xattn.k.weight", "head.xattn.k.bias", D, D, h.k, true) &&
             L.linear("head.xattn.v.weight", "head.xattn.v.bias", D, D, h.v, true) &&
             L.linear("head.xattn.ffn_up.weight", "head.xattn.ffn_up.bias", D, Fx, h.up, true) &&
             L.linear("head.xattn.ffn_down.weight", "head.xattn.ffn_down.bias", Fx, D, h.down, true) &&
             L.linear("head.cls.weight", "head.cls.bias", D, C, h.cls, true, true);
        if (ok && m->hp.n_classes > 0 && C != m->hp.n_classes) {
            jepa_log("jepa: head.cls.weight has %" PRId64 " rows, jepa.head.n_classes is %d\n", C, m->hp.n_classes);
            ok = false;
        }
    }
    if (L.staging) hipFree(L.staging);
    hipStreamDestroy(s);
    if (!ok) {
        model_free_device(m.get());
        return nullptr;
    }
    if (mp.verbose) {
        hipDeviceProp_t prop;
        hipGetDeviceProperties(&prop, device);
        jepa_log("jepa: loaded %s: family=%s name='%s' ftype=%s D=%d L=%d H=%d ffn=%d patch=%d tubelet=%d img=%d on HIP%d (%s), "
                 "%.1f MiB of device weights\n", path, m->hp.family_str.c_str(), m->hp.name.c_str(), jepa_file_type_name_u32(m->hp.file_type),
                 e.embed_dim, e.n_layer, e.n_head, e.ffn_dim, e.patch_size, e.tubelet_size, e.img_size, device, prop.name,
                 m->n_bytes_weights / 1048576.0);
    }
    return m.release();
}
