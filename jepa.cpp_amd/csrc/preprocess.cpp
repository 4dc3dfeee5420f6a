// preprocess.cpp - host image / video preprocessing behind include/jepa.h (reference src/preprocess.cpp).
//
// jepa_resize_antialias_u8 is the uint8 antialiased resize that torchvision's resize(antialias=True)
// runs on CPU (PyTorch's separable uint8 bilinear / bicubic kernel, Pillow's ImagingResample method),
// which the reference reproduces (src/preprocess.cpp:1-10) and whose outputs these functions must equal
// bit for bit:
//   - separable: the horizontal pass first, rounded to uint8, then the vertical pass;
//   - per output position, filter taps over the input window [center - support, center + support),
//     support = (taps / 2) * max(scale, 1), the filter argument scaled by 1 / max(scale, 1)
//     (triangle for bilinear, Keys cubic a = -0.5 for bicubic), weights normalised in double;
//   - weights quantised to int16 with the largest precision whose largest weight still fits 15 bits;
//     int32 accumulation from a rounding offset of 2^(precision-1), output clamp(acc >> precision).
// Then the centre crop (zero padding when the image is smaller than the crop) and the mean / std
// normalisation into NCTHW floats. The same tables drive the device version (preprocess.hip).
#include "model.h"
#include "preprocess.h"

#include <zlib.h>

#include <algorithm>
#include <cmath>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <vector>

namespace {

double tri(double x) {
    x = std::fabs(x);
    return x < 1.0 ? 1.0 - x : 0.0;
}

// Keys cubic convolution kernel with a = -0.5, in the Horner form of its two pieces
double keys_cubic(double x) {
    const double a = -0.5;
    x = std::fabs(x);
    if (x < 1.0) return ((a + 2.0) * x - (a + 3.0)) * x * x + 1.0;
    if (x < 2.0) return ((a * x - 5.0 * a) * x + 8.0 * a) * x - 4.0 * a;
    return 0.0;
}

}  // namespace

aa_taps aa_taps_for(int in_size, int out_size, int resample) {
    aa_taps t;
    if (in_size <= 0 || out_size <= 0) return t;
    const int taps = resample == JEPA_RESAMPLE_BICUBIC ? 4 : 2;
    double (*filt)(double) = resample == JEPA_RESAMPLE_BICUBIC ? keys_cubic : tri;
    const double scale = (double) in_size / (double) out_size;
    const double support = scale >= 1.0 ? (taps * 0.5) * scale : taps * 0.5;
    const double fscale = scale >= 1.0 ? 1.0 / scale : 1.0;
    t.ksize = (int) std::ceil(support) * 2 + 1;
    t.first.assign((size_t) out_size, 0);
    t.count.assign((size_t) out_size, 0);
    std::vector<double> wd((size_t) out_size * t.ksize, 0.0);
    double wmax = 0.0;
    for (int i = 0; i < out_size; i++) {
        const double center = scale * (i + 0.5);
        const int64_t lo = std::max<int64_t>((int64_t) (center - support + 0.5), 0);
        int64_t n = std::min<int64_t>((int64_t) (center + support + 0.5), in_size) - lo;
        n = std::min<int64_t>(std::max<int64_t>(n, 0), t.ksize);
        double * w = wd.data() + (size_t) i * t.ksize;
        double sum = 0.0;
        for (int64_t j = 0; j < n; j++) {
            w[j] = filt((j + lo - center + 0.5) * fscale);
            sum += w[j];
        }
        if (sum != 0.0)
            for (int64_t j = 0; j < n; j++) {
                w[j] /= sum;
                wmax = std::max(wmax, w[j]);
            }
        t.first[(size_t) i] = (int) lo;
        t.count[(size_t) i] = (int) n;
    }
    int prec = 0;
    while (prec < 22 && (int) (0.5 + wmax * (double) (1 << (prec + 1))) < (1 << 15)) prec++;
    t.precision = prec;
    t.w.assign(wd.size(), 0);
    for (size_t j = 0; j < wd.size(); j++) {
        const double v = wd[j] * (double) (1 << prec);
        t.w[j] = (int16_t) (v < 0 ? (int) (-0.5 + v) : (int) (0.5 + v));
    }
    return t;
}

static inline uint8_t clamp_shift(int32_t acc, int prec) {
    const int32_t v = acc >> prec;
    return (uint8_t) (v < 0 ? 0 : v > 255 ? 255 : v);
}

extern "C" void jepa_resize_antialias_u8(const uint8_t * src, int h, int w, int c, uint8_t * dst, int out_h, int out_w, int resample) {
    if (!src || !dst || h <= 0 || w <= 0 || c <= 0 || out_h <= 0 || out_w <= 0) {
        jepa_log("jepa: jepa_resize_antialias_u8: %dx%dx%d -> %dx%d is not a resize\n", h, w, c, out_h, out_w);
        return;
    }
    if (h == out_h && w == out_w) {
        memcpy(dst, src, (size_t) h * w * c);
        return;
    }
    std::vector<uint8_t> mid;
    const uint8_t * rows = src;
    int rw = w;
    if (out_w != w) {   // horizontal pass (into dst directly when there is no vertical one)
        const aa_taps t = aa_taps_for(w, out_w, resample);
        const int32_t bias = t.precision > 0 ? 1 << (t.precision - 1) : 0;
        uint8_t * o = out_h == h ? dst : (mid.resize((size_t) h * out_w * c), mid.data());
        for (int y = 0; y < h; y++) {
            const uint8_t * in = src + (size_t) y * w * c;
            uint8_t * orow = o + (size_t) y * out_w * c;
            for (int x = 0; x < out_w; x++) {
                const int16_t * k = t.w.data() + (size_t) x * t.ksize;
                const uint8_t * p = in + (size_t) t.first[(size_t) x] * c;
                for (int ch = 0; ch < c; ch++) {
                    int32_t acc = bias;
                    for (int j = 0; j < t.count[(size_t) x]; j++) acc += (int32_t) p[(size_t) j * c + ch] * k[j];
                    orow[(size_t) x * c + ch] = clamp_shift(acc, t.precision);
                }
            }
        }
        if (out_h == h) return;
        rows = mid.data();
        rw = out_w;
    }
    const aa_taps t = aa_taps_for(h, out_h, resample);   // vertical pass
    const int32_t bias = t.precision > 0 ? 1 << (t.precision - 1) : 0;
    const size_t rowlen = (size_t) rw * c;
    std::vector<int32_t> acc(rowlen);
    for (int y = 0; y < out_h; y++) {
        const int16_t * k = t.w.data() + (size_t) y * t.ksize;
        std::fill(acc.begin(), acc.end(), bias);
        for (int j = 0; j < t.count[(size_t) y]; j++) {
            const uint8_t * r = rows + (size_t) (t.first[(size_t) y] + j) * rowlen;
            const int32_t kj = k[j];
            for (size_t i = 0; i < rowlen; i++) acc[i] += (int32_t) r[i] * kj;
        }
        uint8_t * orow = dst + (size_t) y * rowlen;
        for (size_t i = 0; i < rowlen; i++) orow[i] = clamp_shift(acc[i], t.precision);
    }
}

// ------------------------------------------------------------------------------------------------
// geometry and normalisation shared with the device path
// ------------------------------------------------------------------------------------------------
bool pre_plan_for(const jepa_preprocess_params * p, int h, int w, pre_plan & g) {
    if (!p) return false;
    if (p->resize_short <= 0) {
        jepa_log("jepa: preprocess: resize_short is %d - nothing to resize to\n", p->resize_short);
        return false;
    }
    for (int c = 0; c < 3; c++) {
        if (!(p->std[c] > 1e-9f) || !(p->std[c] < 1e9f) || !(p->rescale > 0.0f)) {
            jepa_log("jepa: preprocess: std[%d] = %g and rescale = %g must be finite and non-zero\n", c, (double) p->std[c],
                     (double) p->rescale);
            return false;
        }
    }
    // shortest edge to resize_short keeping the aspect ratio (integer floor on the long side), or a
    // square squash (reference src/preprocess.cpp:202-216)
    int64_t rh, rw;
    if (p->resize_mode == JEPA_RESIZE_SQUASH) {
        rh = rw = p->resize_short;
    } else if (w <= h) {
        rw = p->resize_short;
        rh = (int64_t) p->resize_short * h / w;
    } else {
        rh = p->resize_short;
        rw = (int64_t) p->resize_short * w / h;
    }
    rh = std::max<int64_t>(rh, 1);
    rw = std::max<int64_t>(rw, 1);
    if (rh * rw > JEPA_PRE_MAX_PIXELS) {
        jepa_log("jepa: preprocess: %dx%d at shortest edge %d resizes to %lldx%lld = %.1f megapixels, over the %lld-megapixel "
                 "limit (the aspect ratio makes this buffer large)\n",
                 h, w, p->resize_short, (long long) rh, (long long) rw, (double) (rh * rw) / 1048576.0,
                 (long long) (JEPA_PRE_MAX_PIXELS >> 20));
        return false;
    }
    g.rh = (int) rh;
    g.rw = (int) rw;
    g.crop = p->crop > 0 ? p->crop : std::min(g.rh, g.rw);
    // centre crop of the (zero-padded when smaller) resized image: crop pixel (y, x) is resized pixel
    // (y + oy, x + ox), outside [0, rh) x [0, rw) it is a zero pixel
    const int pt = g.crop > g.rh ? (g.crop - g.rh) / 2 : 0, pl = g.crop > g.rw ? (g.crop - g.rw) / 2 : 0;
    const int nh = std::max(g.crop, g.rh), nw = std::max(g.crop, g.rw);
    g.oy = (nh - g.crop) / 2 - pt;
    g.ox = (nw - g.crop) / 2 - pl;
    // the float32 1/rescale (255 for 1/255) snapped to an integer when it is one up to rounding,
    // as the HF processors' double inversion gives (reference src/preprocess.cpp:256-260)
    double inv = 1.0 / (double) p->rescale;
    if (std::fabs(inv - std::nearbyint(inv)) < 1e-3 * std::fabs(inv)) inv = std::nearbyint(inv);
    g.inv = (float) inv;
    g.fused = p->fused_norm;
    for (int c = 0; c < 3; c++) {
        g.mean[c] = g.fused ? p->mean[c] * g.inv : p->mean[c];
        g.stdv[c] = g.fused ? p->std[c] * g.inv : p->std[c];
    }
    return true;
}

extern "C" float * jepa_preprocess_frames_rgb_ex(const jepa_preprocess_params * p, const uint8_t * const * frames, int n_frames, int h,
                                                 int w, int * out_h, int * out_w) {
    if (!p || !frames || n_frames <= 0 || h <= 0 || w <= 0) return nullptr;
    if ((double) h * w * 3 >= (double) SIZE_MAX) {
        jepa_log("jepa: preprocess: a %dx%d RGB frame cannot be a buffer\n", h, w);
        return nullptr;
    }
    pre_plan g;
    if (!pre_plan_for(p, h, w, g)) return nullptr;
    const size_t plane = (size_t) g.crop * g.crop;
    if ((double) 3 * n_frames * plane * sizeof(float) >= (double) SIZE_MAX) {
        jepa_log("jepa: preprocess: %d frames of %dx%d floats do not fit in memory\n", n_frames, g.crop, g.crop);
        return nullptr;
    }
    float * out = (float *) malloc((size_t) 3 * n_frames * plane * sizeof(float));
    if (!out) return nullptr;
    std::vector<uint8_t> rs((size_t) g.rh * g.rw * 3);
    for (int t = 0; t < n_frames; t++) {
        if (!frames[t]) { free(out); return nullptr; }
        jepa_resize_antialias_u8(frames[t], h, w, 3, rs.data(), g.rh, g.rw, p->resample);
        for (int c = 0; c < 3; c++) {
            float * dst = out + ((size_t) c * n_frames + t) * plane;
            for (int y = 0; y < g.crop; y++) {
                const int sy = y + g.oy;
                for (int x = 0; x < g.crop; x++) {
                    const int sx = x + g.ox;
                    const uint8_t v = (sy >= 0 && sy < g.rh && sx >= 0 && sx < g.rw) ? rs[((size_t) sy * g.rw + sx) * 3 + c] : 0;
                    dst[(size_t) y * g.crop + x] = pre_normalize(g, c, v);
                }
            }
        }
    }
    if (out_h) *out_h = g.crop;
    if (out_w) *out_w = g.crop;
    return out;
}

extern "C" float * jepa_preprocess_image_rgb_ex(const jepa_preprocess_params * p, const uint8_t * rgb, int h, int w, int * out_h, int * out_w) {
    const uint8_t * frames[1] = {rgb};
    return jepa_preprocess_frames_rgb_ex(p, frames, 1, h, w, out_h, out_w);
}

extern "C" float * jepa_preprocess_frames_rgb(const jepa_model * model, const uint8_t * const * frames, int n_frames, int h, int w,
                                              int * out_h, int * out_w) {
    const jepa_preprocess_params p = jepa_preprocess_default_params(model);
    return jepa_preprocess_frames_rgb_ex(&p, frames, n_frames, h, w, out_h, out_w);
}

extern "C" float * jepa_preprocess_image_rgb(const jepa_model * model, const uint8_t * rgb, int h, int w, int * out_h, int * out_w) {
    const jepa_preprocess_params p = jepa_preprocess_default_params(model);
    return jepa_preprocess_image_rgb_ex(&p, rgb, h, w, out_h, out_w);
}

extern "C" float * jepa_preprocess_image_file(const jepa_model * model, const char * path, int * out_h, int * out_w) {
    int h = 0, w = 0;
    uint8_t * rgb = jepa_load_image_rgb(path, &h, &w);
    if (!rgb) return nullptr;
    float * out = jepa_preprocess_image_rgb(model, rgb, h, w, out_h, out_w);
    free(rgb);
    return out;
}
