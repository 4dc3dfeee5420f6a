// preprocess.cpp - host image / video preprocessing behind include/jepa.h (reference src/preprocess.cpp).
//
// The resize is the uint8 antialiased resample that torchvision's resize(antialias=True) runs on
// the CPU (PyTorch's separable uint8 kernel, which implements Pillow's ImagingResample), and whose
// bytes the reference reproduces (src/preprocess.cpp:1-10). What that method fixes, and this file
// therefore keeps:
//   - the filter: triangle (bilinear, radius 1) or Keys' cubic with a = -0.5 (bicubic, radius 2),
//     stretched by the downscale factor, evaluated in double at (input index - centre + 0.5) with
//     centre = scale * (output index + 0.5), over the inputs whose rounded window
//     [centre - radius, centre + radius) covers them; each output's weights divided by their sum;
//   - int16 taps: the weights times 2^shift rounded half away from zero, shift the largest value
//     (at most 22) at which the largest weight still rounds below 2^15 one step later;
//   - integer accumulation from 2^(shift-1), result clamp(acc >> shift, 0, 255);
//   - the horizontal pass first, its uint8 result fed to the vertical pass; a pass whose size does
//     not change is skipped (its taps would be the identity).
// The tables are compressed rows (resample_axis): every output keeps only its own taps, and the
// device passes (preprocess.hip) read the same arrays.
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

// the two antialias filters, each with its radius at scale 1
struct aa_filter {
    double radius;
    double (*at)(double);
};

double triangle_at(double x) {
    const double d = std::fabs(x);
    return d < 1.0 ? 1.0 - d : 0.0;
}

// Keys (1981) cubic convolution, a = -0.5, in the nested form torch evaluates (the weights must be
// the same doubles for the int16 rounding to agree): inner piece ((a+2)|x| - (a+3))|x|^2 + 1,
// outer piece ((a|x| - 5a)|x| + 8a)|x| - 4a
double keys_at(double x) {
    constexpr double a = -0.5;
    const double d = std::fabs(x);
    if (d >= 2.0) return 0.0;
    if (d >= 1.0) return ((a * d - 5.0 * a) * d + 8.0 * a) * d - 4.0 * a;
    return ((a + 2.0) * d - (a + 3.0)) * d * d + 1.0;
}

// round half away from zero the way the method writes it, (int)(0.5 + |v|) with the sign put back
int16_t round_tap(double v) {
    const int mag = (int) (0.5 + std::fabs(v));
    return (int16_t) (v < 0.0 ? -mag : mag);
}

uint8_t settle(int32_t acc, int shift) {
    const int32_t v = acc >> shift;
    return (uint8_t) std::min<int32_t>(255, std::max<int32_t>(0, v));
}

// horizontal pass: every row of `rows` (height h, n_in pixels of c channels) into n_out pixels
void resample_rows(const resample_axis & ax, const uint8_t * src, int h, int c, uint8_t * dst) {
    const int32_t half = ax.shift > 0 ? (int32_t) 1 << (ax.shift - 1) : 0;
    std::vector<int32_t> acc((size_t) c);
    for (int y = 0; y < h; y++) {
        const uint8_t * in = src + (size_t) y * ax.n_in * c;
        uint8_t * out = dst + (size_t) y * ax.n_out * c;
        for (int o = 0; o < ax.n_out; o++) {
            std::fill(acc.begin(), acc.end(), half);
            const uint8_t * px = in + (size_t) ax.lo[(size_t) o] * c;
            for (int32_t t = ax.beg[(size_t) o]; t < ax.beg[(size_t) o + 1]; t++, px += c) {
                const int32_t tap = ax.taps[(size_t) t];
                for (int ch = 0; ch < c; ch++) acc[(size_t) ch] += tap * (int32_t) px[ch];
            }
            for (int ch = 0; ch < c; ch++) out[(size_t) o * c + ch] = settle(acc[(size_t) ch], ax.shift);
        }
    }
}

// vertical pass: rows of `len` bytes, n_in of them, into n_out rows (whole rows scaled and summed)
void resample_cols(const resample_axis & ax, const uint8_t * src, size_t len, uint8_t * dst) {
    const int32_t half = ax.shift > 0 ? (int32_t) 1 << (ax.shift - 1) : 0;
    std::vector<int32_t> acc(len);
    for (int o = 0; o < ax.n_out; o++) {
        std::fill(acc.begin(), acc.end(), half);
        const uint8_t * row = src + (size_t) ax.lo[(size_t) o] * len;
        for (int32_t t = ax.beg[(size_t) o]; t < ax.beg[(size_t) o + 1]; t++, row += len) {
            const int32_t tap = ax.taps[(size_t) t];
            for (size_t i = 0; i < len; i++) acc[i] += tap * (int32_t) row[i];
        }
        uint8_t * out = dst + (size_t) o * len;
        for (size_t i = 0; i < len; i++) out[i] = settle(acc[i], ax.shift);
    }
}

}  // namespace

resample_axis resample_axis_for(int n_in, int n_out, int resample) {
    resample_axis ax;
    if (n_in <= 0 || n_out <= 0) return ax;
    ax.n_in = n_in;
    ax.n_out = n_out;
    const aa_filter f = resample == JEPA_RESAMPLE_BICUBIC ? aa_filter{2.0, keys_at} : aa_filter{1.0, triangle_at};
    const double scale = (double) n_in / (double) n_out;
    const double stretch = std::max(scale, 1.0);        // the filter widens only when shrinking
    const double reach = f.radius * stretch;
    const double step = 1.0 / stretch;
    ax.lo.resize((size_t) n_out);
    ax.beg.assign(1, 0);
    std::vector<double> weight;
    double peak = 0.0;
    for (int o = 0; o < n_out; o++) {
        const double centre = scale * (o + 0.5);
        // inputs whose window rounds into [centre - reach, centre + reach), clipped to the image (in
        // double before the conversion, so that a very wide input cannot push it past INT_MAX)
        const int first = (int) std::max(0.0, centre - reach + 0.5);
        const int end = (int) std::min((double) n_in, centre + reach + 0.5);
        const size_t row0 = weight.size();
        double total = 0.0;
        for (int x = first; x < end; x++) {
            const double v = f.at((x - centre + 0.5) * step);
            weight.push_back(v);
            total += v;
        }
        if (total != 0.0)
            for (size_t t = row0; t < weight.size(); t++) {
                weight[t] /= total;
                peak = std::max(peak, weight[t]);
            }
        ax.lo[(size_t) o] = first;
        ax.beg.push_back((int32_t) weight.size());
    }
    // shift: the first s in 0..21 whose next step would round the peak weight to 2^15 or more,
    // else 22
    ax.shift = 22;
    for (int s = 0; s < 22; s++)
        if ((int) (0.5 + peak * (double) (1 << (s + 1))) >= (1 << 15)) { ax.shift = s; break; }
    ax.taps.resize(weight.size());
    const double unit = (double) (1 << ax.shift);
    for (size_t t = 0; t < weight.size(); t++) ax.taps[t] = round_tap(weight[t] * unit);
    return ax;
}

extern "C" void jepa_resize_antialias_u8(const uint8_t * src, int h, int w, int c, uint8_t * dst, int out_h, int out_w, int resample) {
    if (!src || !dst || h <= 0 || w <= 0 || c <= 0 || out_h <= 0 || out_w <= 0) {
        jepa_log("jepa: jepa_resize_antialias_u8: %dx%dx%d -> %dx%d is not a resize\n", h, w, c, out_h, out_w);
        return;
    }
    const bool across = out_w != w, down = out_h != h;
    if (!across && !down) {
        memcpy(dst, src, (size_t) h * w * c);
        return;
    }
    // the horizontal result goes straight to dst when it is the last pass
    std::vector<uint8_t> between;
    const uint8_t * vin = src;
    if (across) {
        uint8_t * hout = dst;
        if (down) {
            between.resize((size_t) h * out_w * c);
            hout = between.data();
        }
        resample_rows(resample_axis_for(w, out_w, resample), src, h, c, hout);
        vin = hout;
    }
    if (down) resample_cols(resample_axis_for(h, out_h, resample), vin, (size_t) out_w * c, dst);
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
    // each side first: a large resize_short at an extreme aspect ratio would overflow the product
    if (rh > JEPA_PRE_MAX_PIXELS || rw > JEPA_PRE_MAX_PIXELS || rh * rw > JEPA_PRE_MAX_PIXELS) {
        jepa_log("jepa: preprocess: %dx%d at shortest edge %d resizes to %lldx%lld = %.1f megapixels, over the %lld-megapixel "
                 "limit (the aspect ratio makes this buffer large)\n",
                 h, w, p->resize_short, (long long) rh, (long long) rw, (double) rh * (double) rw / 1048576.0,
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
