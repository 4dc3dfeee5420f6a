// api.cpp - the encoder-path entry points of include/jepa.h: diagnostics, devices, contexts,
// jepa_encode, pooling, introspection, small host helpers.
//
// Behaviour follows reference src/jepa.cpp (error conventions 16-36, device parsing 107-132,
// context knobs 178-254, encode dispatch and input checks 1183-1224, pooling 1229-1271, softmax /
// top-k 1134-1156, token grid 1158-1181) and src/jepa-gguf.cpp:1122-1152 (introspection).
#include "model.h"

#include <algorithm>
#include <atomic>
#include <cctype>
#include <cmath>
#include <cstdarg>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <mutex>
#include <string>
#include <thread>
#include <vector>

// ---------------------------------------------------------------------------------------------
// diagnostics (reference src/jepa.cpp:16-36)
// ---------------------------------------------------------------------------------------------
static const size_t JEPA_ERROR_TEXT_MAX = 8192;
static thread_local std::string g_error_text;

void jepa_log(const char * fmt, ...) {
    va_list ap;
    va_start(ap, fmt);
    vfprintf(stderr, fmt, ap);
    va_end(ap);
    if (g_error_text.size() >= JEPA_ERROR_TEXT_MAX) return;
    char buf[1024];
    va_list ap2;
    va_start(ap2, fmt);
    const int n = vsnprintf(buf, sizeof(buf), fmt, ap2);
    va_end(ap2);
    if (n <= 0) return;
    g_error_text.append(buf, std::min((size_t) n, sizeof(buf) - 1));
    if (g_error_text.size() > JEPA_ERROR_TEXT_MAX) g_error_text.resize(JEPA_ERROR_TEXT_MAX);
}

extern "C" void jepa_error_reset(void) { g_error_text.clear(); }
extern "C" const char * jepa_error_text(void) { return g_error_text.c_str(); }
extern "C" const char * jepa_version(void) { return JEPA_VERSION; }

// ---------------------------------------------------------------------------------------------
// devices: HIP devices in runtime order; -1 (the reference's "CPU") resolves to device 0, since this
// library computes on a GPU and has no CPU path
// ---------------------------------------------------------------------------------------------
namespace {
struct device_info { std::string name, description; };
const std::vector<device_info> & devices() {
    static std::vector<device_info> v = [] {
        std::vector<device_info> out;
        int n = 0;
        if (hipGetDeviceCount(&n) != hipSuccess) { hipGetLastError(); n = 0; }
        for (int i = 0; i < n; i++) {
            hipDeviceProp_t p;
            device_info d;
            d.name = "HIP" + std::to_string(i);
            d.description = hipGetDeviceProperties(&p, i) == hipSuccess ? std::string(p.name) : std::string("HIP device");
            out.push_back(d);
        }
        return out;
    }();
    return v;
}
}  // namespace

int dev_count() { return (int) devices().size(); }

bool dev_check(int device) {
    const int n = dev_count();
    if (device >= 0 && device < n) return true;
    if (n == 0) jepa_log("jepa: no HIP device is available - this library runs the encoder on an AMD GPU only\n");
    else jepa_log("jepa: GPU device %d does not exist (%d available: 0..%d)\n", device, n, n - 1);
    return false;
}

int dev_resolve(int requested) {
    const int d = requested < 0 ? 0 : requested;
    return dev_check(d) ? d : -1;
}

int device_from_env() {
    const char * s = getenv("JEPA_DEVICE");
    if (!s || !*s) return -1;
    std::string v(s);
    for (char & c : v) c = (char) tolower((unsigned char) c);
    if (v == "cpu") return -1;
    const size_t p = v.find(':');
    const std::string head = p == std::string::npos ? v : v.substr(0, p);
    const std::string tail = p == std::string::npos ? "" : v.substr(p + 1);
    if (head == "cuda" || head == "gpu" || head == "hip" || head == "rocm") {
        const int n = tail.empty() ? 0 : atoi(tail.c_str());
        return n >= 0 ? n : -1;
    }
    if (p == std::string::npos && !v.empty() && v.find_first_not_of("0123456789") == std::string::npos) return atoi(v.c_str());
    static std::atomic<bool> warned{false};
    if (!warned.exchange(true)) jepa_log("jepa: ignoring JEPA_DEVICE='%s' (expected cpu, gpu:N, hip:N or a bare device index)\n", s);
    return -1;
}

extern "C" int jepa_device_count(void) { return dev_count(); }
extern "C" const char * jepa_device_name(int device) { return dev_check(device) ? devices()[(size_t) device].name.c_str() : nullptr; }
extern "C" const char * jepa_device_description(int device) {
    return dev_check(device) ? devices()[(size_t) device].description.c_str() : nullptr;
}
extern "C" void jepa_device_memory(int device, size_t * free_bytes, size_t * total_bytes) {
    size_t f = 0, t = 0;
    if (dev_check(device)) {
        int prev = 0;
        hipGetDevice(&prev);
        hipSetDevice(device);
        if (hipMemGetInfo(&f, &t) != hipSuccess) { f = t = 0; hipGetLastError(); }
        hipSetDevice(prev);
    }
    if (free_bytes) *free_bytes = f;
    if (total_bytes) *total_bytes = t;
}
extern "C" int jepa_model_device(const jepa_model * m) { return m ? m->device : -1; }
extern "C" bool jepa_model_is_gpu(const jepa_model * m) { return m != nullptr; }
extern "C" const char * jepa_model_device_name(const jepa_model * m) { return m ? jepa_device_name(m->device) : nullptr; }

extern "C" void jepa_print_system_info(void) {
    fprintf(stderr, "jepa.cpp-mi355x %s | HIP | devices: %d", JEPA_VERSION, dev_count());
    for (int i = 0; i < dev_count(); i++) fprintf(stderr, " | %s: %s", devices()[(size_t) i].name.c_str(), devices()[(size_t) i].description.c_str());
    fprintf(stderr, "\n");
}

// ---------------------------------------------------------------------------------------------
// contexts (reference src/jepa.cpp:178-254)
// ---------------------------------------------------------------------------------------------
extern "C" jepa_context_params jepa_context_default_params(void) {
    jepa_context_params p;
    p.n_threads = 0;
    p.use_flash_attn = true;
    p.verbose = false;
    p.flash_kv = JEPA_KV_AUTO;
    return p;
}

extern "C" jepa_context * jepa_context_new(jepa_model * model, jepa_context_params params) {
    if (!model) return nullptr;
    std::unique_ptr<jepa_context> ctx(new jepa_context());
    ctx->model = model;
    ctx->params = params;
    ctx->n_threads = params.n_threads > 0 ? params.n_threads : (int) std::thread::hardware_concurrency();
    if (ctx->n_threads < 1) ctx->n_threads = 1;
    ctx->device = model->device;
    if (hipSetDevice(ctx->device) != hipSuccess || hipStreamCreateWithFlags(&ctx->stream, hipStreamNonBlocking) != hipSuccess ||
        hipEventCreate(&ctx->ev0) != hipSuccess || hipEventCreate(&ctx->ev1) != hipSuccess) {
        jepa_log("jepa: could not create a HIP stream / events on device %d\n", ctx->device);
        return nullptr;
    }
    if (params.flash_kv == JEPA_KV_F32) {
        static std::atomic<bool> warned{false};
        if (!warned.exchange(true))
            jepa_log("jepa: F32 K/V was requested but the attention kernel holds K/V in f16 (as the reference's GPU path does)\n");
    }
    if (!params.use_flash_attn) {
        static std::atomic<bool> warned{false};
        if (!warned.exchange(true)) jepa_log("jepa: use_flash_attn = false: the fused attention kernel is the only attention path here\n");
    }
    if (const char * s = getenv("JEPA_MAX_BATCH")) { const int v = atoi(s); if (v > 0) ctx->max_batch = v; }
    if (const char * s = getenv("JEPA_MAX_GRAPH_MIB")) { const long long v = atoll(s); if (v > 0) ctx->max_graph_bytes = (size_t) v << 20; }
    if (const char * s = getenv("JEPA_HIP_GRAPH")) ctx->use_graph = atoi(s) != 0;
    return ctx.release();
}

extern "C" void jepa_context_free(jepa_context * ctx) { delete ctx; }
extern "C" int jepa_context_n_threads(const jepa_context * ctx) { return ctx ? ctx->n_threads : 0; }
extern "C" double jepa_context_last_compute_ms(const jepa_context * ctx) { return ctx ? ctx->last_compute_ms : 0.0; }
extern "C" void jepa_context_set_max_batch(jepa_context * ctx, int n) { if (ctx) ctx->max_batch = n > 0 ? n : 0; }
extern "C" int jepa_context_max_batch(const jepa_context * ctx) {
    if (!ctx) return 0;
    return ctx->max_batch > 0 ? ctx->max_batch : JEPA_DEFAULT_MAX_BATCH;
}
extern "C" int jepa_context_last_batch(const jepa_context * ctx) { return ctx ? ctx->last_batch : 0; }
extern "C" void jepa_context_set_mul_mat_prec_f32(jepa_context * ctx, bool on) { if (ctx) ctx->prec_f32 = on; }
extern "C" bool jepa_context_mul_mat_prec_f32(const jepa_context * ctx) { return ctx && ctx->prec_f32; }

// ---------------------------------------------------------------------------------------------
// jepa_encode (reference src/jepa.cpp:1183-1224)
// ---------------------------------------------------------------------------------------------
extern "C" int jepa_encode(jepa_context * ctx, const jepa_input * in, jepa_output * out) {
    if (!ctx || !in || !out || !in->data) return -1;
    const jepa_model * m = ctx->model;
    if (in->n_chans != m->hp.enc.in_chans) {
        jepa_log("jepa: input has %d channels, model expects %d\n", in->n_chans, m->hp.enc.in_chans);
        return -1;
    }
    if (in->n_batch < 1 || in->n_frames < 1 || in->height < 1 || in->width < 1) {
        jepa_log("jepa: bad input shape [%d, %d, %d, %d, %d]\n", in->n_batch, in->n_chans, in->n_frames, in->height, in->width);
        return -1;
    }
    const double n_elems = (double) in->n_batch * in->n_chans * in->n_frames * in->height * in->width;
    if (n_elems * sizeof(float) >= (double) SIZE_MAX) {
        jepa_log("jepa: input shape [%d, %d, %d, %d, %d] describes %.3g floats, which cannot be a buffer\n", in->n_batch, in->n_chans,
                 in->n_frames, in->height, in->width, n_elems);
        return -1;
    }
    out->data = nullptr; out->n_tokens = 0; out->dim = 0;
    int64_t n_items = 0;
    const int64_t R = encode_rows(m, in->n_batch, in->n_frames, in->height, in->width, &n_items);
    const int64_t D = m->hp.enc.embed_dim;
    if (R <= 0) {
        // reuse the device path's diagnostics for the exact reason
        encode_host(ctx, in, nullptr, 0);
        return -1;
    }
    if ((double) n_items * (double) R * (double) D * sizeof(float) >= (double) SIZE_MAX) {
        jepa_log("jepa: %lld items x %lld tokens x %lld dims does not fit in memory\n", (long long) n_items, (long long) R, (long long) D);
        return -1;
    }
    float * data = (float *) malloc((size_t) n_items * R * D * sizeof(float));
    if (!data) {
        jepa_log("jepa: could not allocate %.1f MiB for %lld output rows\n", (double) n_items * R * D * 4 / 1048576.0, (long long) (n_items * R));
        return -1;
    }
    if (encode_host(ctx, in, data, n_items * R * D) < 0) { free(data); return -1; }
    out->data = data;
    out->n_tokens = n_items * R;
    out->dim = D;
    return 0;
}

extern "C" int64_t jepa_token_grid(const jepa_model * model, int n_frames, int height, int width, int * gt, int * gh, int * gw) {
    if (!model || n_frames < 1 || height < 1 || width < 1) return 0;
    if (is_video_family(model->hp.family)) {
        video_shape vs;
        if (!video_shape_for(model, n_frames, height, width, vs, false)) return 0;
        if (gt) *gt = vs.gt;
        if (gh) *gh = vs.gh;
        if (gw) *gw = vs.gw;
        return vs.n_rows();
    }
    if (model->hp.family == FAM_VJEPA) {
        jepa_log("jepa: jepa_token_grid: family '%s' is not implemented on this path\n", model->hp.family_str.c_str());
        return 0;
    }
    const enc_hparams & e = model->hp.enc;
    if (e.patch_size <= 0 || height % e.patch_size || width % e.patch_size) return 0;
    if (gt) *gt = n_frames;
    if (gh) *gh = height / e.patch_size;
    if (gw) *gw = width / e.patch_size;
    return (int64_t) n_frames * ((int64_t) (height / e.patch_size) * (width / e.patch_size) + (e.cls_token ? 1 : 0) + e.n_registers);
}

// ---------------------------------------------------------------------------------------------
// pooling (reference src/jepa.cpp:1229-1271), host side
// ---------------------------------------------------------------------------------------------
extern "C" int jepa_pool_mean(const jepa_model * model, const jepa_output * enc, jepa_output * out) {
    if (!model || !enc || !out || !enc->data) return -1;
    const int64_t skip = (model->hp.enc.cls_token ? 1 : 0) + model->hp.enc.n_registers;
    const int64_t D = enc->dim, n = enc->n_tokens - skip;
    if (D <= 0 || enc->n_tokens <= 0) {
        jepa_log("jepa: jepa_pool_mean: encoder output is [%lld tokens, %lld dims]\n", (long long) enc->n_tokens, (long long) D);
        return -1;
    }
    if (n <= 0) return -1;
    out->n_tokens = 1;
    out->dim = D;
    out->data = (float *) calloc((size_t) D, sizeof(float));
    if (!out->data) return -1;
    std::vector<double> acc((size_t) D, 0.0);
    for (int64_t i = skip; i < enc->n_tokens; i++) {
        const float * row = enc->data + i * D;
        for (int64_t d = 0; d < D; d++) acc[(size_t) d] += row[d];
    }
    for (int64_t d = 0; d < D; d++) out->data[d] = (float) (acc[(size_t) d] / (double) n);
    return 0;
}

extern "C" int jepa_pool_cls(const jepa_model * model, const jepa_output * enc, jepa_output * out) {
    if (!model || !enc || !out || !enc->data) return -1;
    if (!model->hp.enc.cls_token) { jepa_log("jepa: jepa_pool_cls: model has no CLS token\n"); return -1; }
    if (enc->dim <= 0 || enc->n_tokens < 1) {
        jepa_log("jepa: jepa_pool_cls: encoder output is [%lld tokens, %lld dims]\n", (long long) enc->n_tokens, (long long) enc->dim);
        return -1;
    }
    out->n_tokens = 1;
    out->dim = enc->dim;
    out->data = (float *) malloc((size_t) enc->dim * sizeof(float));
    if (!out->data) return -1;
    memcpy(out->data, enc->data, (size_t) enc->dim * sizeof(float));
    return 0;
}

// ---------------------------------------------------------------------------------------------
// host helpers (reference src/jepa.cpp:1134-1156)
// ---------------------------------------------------------------------------------------------
extern "C" void jepa_softmax(const float * logits, int n, float * probs) {
    if (n <= 0 || !logits || !probs) return;
    float mx = logits[0];
    for (int i = 1; i < n; i++) mx = logits[i] > mx ? logits[i] : mx;
    double sum = 0;
    for (int i = 0; i < n; i++) { probs[i] = expf(logits[i] - mx); sum += probs[i]; }
    const float inv = (float) (1.0 / (sum > 0 ? sum : 1.0));
    for (int i = 0; i < n; i++) probs[i] *= inv;
}

extern "C" int jepa_top_k(const float * logits, int n, int k, int32_t * idx) {
    if (n <= 0 || k <= 0 || !logits || !idx) return 0;
    if (k > n) k = n;
    std::vector<int32_t> order((size_t) n);
    for (int i = 0; i < n; i++) order[(size_t) i] = i;
    std::partial_sort(order.begin(), order.begin() + k, order.end(),
                      [&](int32_t a, int32_t b) { return logits[a] != logits[b] ? logits[a] > logits[b] : a < b; });
    for (int i = 0; i < k; i++) idx[i] = order[(size_t) i];
    return k;
}

extern "C" void jepa_free(void * p) { free(p); }

// ---------------------------------------------------------------------------------------------
// introspection (reference src/jepa-gguf.cpp:1122-1152)
// ---------------------------------------------------------------------------------------------
extern "C" const char * jepa_model_family(const jepa_model * m) { return m ? m->hp.family_str.c_str() : nullptr; }
extern "C" const char * jepa_model_name(const jepa_model * m) { return m ? m->hp.name.c_str() : nullptr; }
extern "C" int jepa_model_embed_dim(const jepa_model * m) { return m ? m->hp.enc.embed_dim : 0; }
extern "C" int jepa_model_patch_size(const jepa_model * m) { return m ? m->hp.enc.patch_size : 0; }
extern "C" int jepa_model_tubelet_size(const jepa_model * m) { return m ? m->hp.enc.tubelet_size : 0; }
extern "C" int jepa_model_img_size(const jepa_model * m) { return m ? m->hp.enc.img_size : 0; }
extern "C" int jepa_model_n_frames(const jepa_model * m) { return m ? m->hp.enc.n_frames : 0; }
extern "C" int jepa_model_n_layer(const jepa_model * m) { return m ? m->hp.enc.n_layer : 0; }
extern "C" int jepa_model_n_head(const jepa_model * m) { return m ? m->hp.enc.n_head : 0; }
extern "C" bool jepa_model_has_cls(const jepa_model * m) { return m && m->hp.enc.cls_token; }
extern "C" int jepa_model_n_registers(const jepa_model * m) { return m ? m->hp.enc.n_registers : 0; }
extern "C" int jepa_model_n_prefix_tokens(const jepa_model * m) { return m ? (m->hp.enc.cls_token ? 1 : 0) + m->hp.enc.n_registers : 0; }
extern "C" bool jepa_model_has_predictor(const jepa_model * m) { return m && m->hp.has_pred; }
extern "C" bool jepa_model_has_head(const jepa_model * m) { return m && m->hp.has_head; }
extern "C" bool jepa_model_has_projector(const jepa_model * m) { return m && m->hp.enc.has_proj; }
extern "C" int jepa_model_n_classes(const jepa_model * m) { return m ? m->hp.n_classes : 0; }
extern "C" const char * jepa_model_label(const jepa_model * m, int idx) {
    if (!m || idx < 0 || idx >= (int) m->hp.labels.size()) return nullptr;
    return m->hp.labels[(size_t) idx].c_str();
}
extern "C" int jepa_model_file_type(const jepa_model * m) { return m ? (int) m->hp.file_type : -1; }
extern "C" const char * jepa_model_file_type_name(const jepa_model * m) { return m ? jepa_file_type_name_u32(m->hp.file_type) : nullptr; }
extern "C" size_t jepa_model_n_bytes(const jepa_model * m) { return m ? m->n_bytes_weights : 0; }

extern "C" jepa_preprocess_params jepa_preprocess_default_params(const jepa_model * m) {
    jepa_preprocess_params p;
    const pre_hparams def;
    const pre_hparams & s = m ? m->hp.pre : def;
    for (int i = 0; i < 3; i++) { p.mean[i] = s.mean[i]; p.std[i] = s.std[i]; }
    p.resize_short = s.resize_short;
    p.crop = s.crop;
    p.resample = s.resample == "bicubic" ? JEPA_RESAMPLE_BICUBIC : JEPA_RESAMPLE_BILINEAR;
    p.resize_mode = s.resize_mode == "squash" ? JEPA_RESIZE_SQUASH : JEPA_RESIZE_SHORTEST_EDGE;
    p.rescale = s.rescale;
    p.fused_norm = true;
    return p;
}
