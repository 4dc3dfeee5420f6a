// api.cpp - the encoder-path entry points of include/jepa.h: diagnostics, devices, contexts,
// jepa_encode, pooling, introspection, small host helpers.
//
// Behaviour follows the contracts of reference include/jepa.h and src/jepa.cpp (error conventions
// 16-36, device parsing 107-132, context knobs 178-254, encode dispatch and input checks 1183-1224,
// pooling 1229-1271, softmax / top-k 1128-1146, token grid 1158-1181) and src/jepa-gguf.cpp:1122-1152
// (introspection).
#include "model.h"

#include <algorithm>
#include <atomic>
#include <cctype>
#include <cmath>
#include <cstdarg>
#include <cstdint>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <mutex>
#include <string>
#include <thread>
#include <vector>

// ---------------------------------------------------------------------------------------------
// diagnostics: the contract of include/jepa.h:596-610 (every message goes to stderr and into a
// per-thread capture of bounded size that jepa_error_reset empties)
// ---------------------------------------------------------------------------------------------
namespace {
// per-thread capture: a fixed buffer, so logging never allocates on the thread's behalf and a
// runaway caller cannot grow it; once full, later text is dropped (stderr still gets all of it)
struct capture_buffer {
    static constexpr size_t cap = 8192;
    char text[cap + 1] = {0};
    size_t used = 0;
    void clear() { used = 0; text[0] = 0; }
    void add(const char * p, size_t n) {
        const size_t take = std::min(n, cap - used);
        memcpy(text + used, p, take);
        used += take;
        text[used] = 0;
    }
};
thread_local capture_buffer t_capture;
}  // namespace

void jepa_log(const char * fmt, ...) {
    // format once (on the stack for the usual short line, on the heap for a long one), then hand the
    // same bytes to stderr and to the capture
    char small[512];
    va_list ap, again;
    va_start(ap, fmt);
    va_copy(again, ap);
    const int n = vsnprintf(small, sizeof(small), fmt, ap);
    va_end(ap);
    if (n < 0) { va_end(again); return; }
    const char * msg = small;
    std::vector<char> big;
    if ((size_t) n >= sizeof(small)) {
        big.resize((size_t) n + 1);
        vsnprintf(big.data(), big.size(), fmt, again);
        msg = big.data();
    }
    va_end(again);
    fwrite(msg, 1, (size_t) n, stderr);
    t_capture.add(msg, (size_t) n);
}

std::recursive_mutex & jepa_hip_mutex() {
    static std::recursive_mutex mu;
    return mu;
}

extern "C" void jepa_error_reset(void) { t_capture.clear(); }
extern "C" const char * jepa_error_text(void) { return t_capture.text; }
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
    std::lock_guard<std::recursive_mutex> lk(jepa_hip_mutex());
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
namespace {
// The five extents are the only description of in->data: refuse a shape the model cannot take or
// whose element count overflows a byte size, before anything indexes with it (logged refusal).
bool input_acceptable(const jepa_model * m, const jepa_input * in) {
    const int dims[5] = {in->n_batch, in->n_chans, in->n_frames, in->height, in->width};
    if (in->n_chans != m->hp.enc.in_chans) {
        jepa_log("jepa: the model takes %d-channel input; this input has %d channels\n", m->hp.enc.in_chans, in->n_chans);
        return false;
    }
    uint64_t bytes = sizeof(float);
    bool overflow = false;
    for (int d : dims) {
        if (d < 1) {
            jepa_log("jepa: input shape [%d, %d, %d, %d, %d] has an empty extent\n", dims[0], dims[1], dims[2], dims[3], dims[4]);
            return false;
        }
        overflow = overflow || __builtin_mul_overflow(bytes, (uint64_t) d, &bytes);
    }
    if (overflow || bytes > (uint64_t) PTRDIFF_MAX) {
        jepa_log("jepa: input shape [%d, %d, %d, %d, %d] is larger than any buffer can be\n", dims[0], dims[1], dims[2], dims[3],
                 dims[4]);
        return false;
    }
    return true;
}
}  // namespace

extern "C" int jepa_encode(jepa_context * ctx, const jepa_input * in, jepa_output * out) {
    if (!ctx || !in || !out || !in->data) return -1;
    const jepa_model * m = ctx->model;
    if (!input_acceptable(m, in)) return -1;
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
// pooling (contract: include/jepa.h:113-117; reference src/jepa.cpp:1229-1271), host side
// ---------------------------------------------------------------------------------------------
namespace {
// an encoder output the caller filled in: positive extents and data, else a logged refusal
bool pool_input_ok(const char * fn, const jepa_output * enc) {
    if (enc->dim > 0 && enc->n_tokens > 0) return true;
    jepa_log("jepa: %s: encoder output is [%lld tokens, %lld dims]\n", fn, (long long) enc->n_tokens, (long long) enc->dim);
    return false;
}

// one malloc'd row of D floats in out, or false
bool pool_output(jepa_output * out, int64_t D) {
    out->data = (float *) malloc((size_t) D * sizeof(float));
    if (!out->data) {
        out->n_tokens = out->dim = 0;
        return false;
    }
    out->n_tokens = 1;
    out->dim = D;
    return true;
}
}  // namespace

extern "C" int jepa_pool_mean(const jepa_model * model, const jepa_output * enc, jepa_output * out) {
    if (!model || !enc || !out || !enc->data) return -1;
    if (!pool_input_ok("jepa_pool_mean", enc)) return -1;
    // the prefix rows (CLS, registers) are not patches and are left out of the mean
    const int64_t prefix = (int64_t) (model->hp.enc.cls_token ? 1 : 0) + model->hp.enc.n_registers;
    const int64_t rows = enc->n_tokens - prefix, D = enc->dim;
    if (rows <= 0) return -1;
    if (!pool_output(out, D)) return -1;
    // columns in slabs that keep their double partial sums in cache; each sum runs over the rows in
    // order, in double, and is divided once
    constexpr int64_t SLAB = 512;
    double part[SLAB];
    const float * first = enc->data + prefix * D;
    for (int64_t c0 = 0; c0 < D; c0 += SLAB) {
        const int64_t w = std::min(SLAB, D - c0);
        std::fill(part, part + w, 0.0);
        for (int64_t r = 0; r < rows; r++) {
            const float * src = first + r * D + c0;
            for (int64_t c = 0; c < w; c++) part[c] += (double) src[c];
        }
        for (int64_t c = 0; c < w; c++) out->data[c0 + c] = (float) (part[c] / (double) rows);
    }
    return 0;
}

extern "C" int jepa_pool_cls(const jepa_model * model, const jepa_output * enc, jepa_output * out) {
    if (!model || !enc || !out || !enc->data) return -1;
    if (!model->hp.enc.cls_token) {
        jepa_log("jepa: jepa_pool_cls: this model has no CLS token to pool\n");
        return -1;
    }
    if (!pool_input_ok("jepa_pool_cls", enc) || !pool_output(out, enc->dim)) return -1;
    std::copy(enc->data, enc->data + enc->dim, out->data);   // row 0 is the CLS row
    return 0;
}

// ---------------------------------------------------------------------------------------------
// host helpers for classifiers (contract: include/jepa.h:146-150)
// ---------------------------------------------------------------------------------------------
extern "C" void jepa_softmax(const float * logits, int n, float * probs) {
    if (!logits || !probs || n <= 0) return;
    // shifted by the largest logit so that every exponent is <= 0; the normaliser is summed and
    // applied in double
    const float top = *std::max_element(logits, logits + n);
    double total = 0.0;
    for (int i = 0; i < n; i++) {
        probs[i] = expf(logits[i] - top);
        total += (double) probs[i];
    }
    const double scale = total > 0.0 ? 1.0 / total : 1.0;
    for (int i = 0; i < n; i++) probs[i] = (float) ((double) probs[i] * scale);
}

extern "C" int jepa_top_k(const float * logits, int n, int k, int32_t * idx) {
    if (!logits || !idx || n <= 0 || k <= 0) return 0;
    const int want = std::min(k, n);
    // rank: larger logit first, the smaller index on a tie; NaN ranks below every number
    auto before = [logits](int32_t a, int32_t b) {
        const float x = logits[a], y = logits[b];
        const bool xn = std::isnan(x), yn = std::isnan(y);
        if (xn != yn) return yn;
        if (!xn && x != y) return x > y;
        return a < b;
    };
    // a bounded heap of the best `want` seen so far (its top is the weakest member)
    std::vector<int32_t> heap;
    heap.reserve((size_t) want);
    for (int32_t i = 0; i < n; i++) {
        if ((int) heap.size() < want) {
            heap.push_back(i);
            std::push_heap(heap.begin(), heap.end(), before);
        } else if (before(i, heap.front())) {
            std::pop_heap(heap.begin(), heap.end(), before);
            heap.back() = i;
            std::push_heap(heap.begin(), heap.end(), before);
        }
    }
    std::sort_heap(heap.begin(), heap.end(), before);
    std::copy(heap.begin(), heap.end(), idx);
    return want;
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
