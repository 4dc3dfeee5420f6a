// preprocess.hip - uint8 antialiased resize + centre crop + normalisation on the device, equal bit for
// bit to the host jepa_preprocess_frames_rgb_ex (preprocess.cpp; reference src/preprocess.cpp).
//
// The filter tables are built on the host (the double-precision weights and their int16 quantisation
// must be the host's exactly) and uploaded once per call. Two kernels follow the separable order of
// the host resize: the horizontal pass writes only the resized columns the crop keeps, as uint8 (the
// host rounds to uint8 between the passes too); the vertical pass computes the crop's pixels, applies
// the zero padding of an undersized image and writes the normalised floats in NCTHW order.
#include "preprocess.h"

#include <cstring>

namespace {

struct dev_taps {
    const int * first;
    const int * count;
    const int16_t * w;
    int ksize, precision;
    int identity;   // size unchanged: the host skips this pass (a copy)
};

__device__ __forceinline__ uint8_t clamp_shift(int32_t acc, int prec) {
    const int32_t v = acc >> prec;
    return (uint8_t) (v < 0 ? 0 : v > 255 ? 255 : v);
}

// mid[t][y][x][c] = horizontal pass of source row y at resized column x + ox, for the crop columns
// that fall inside the resized image
__global__ void k_resize_rows(const uint8_t * __restrict__ src, uint8_t * __restrict__ mid, int n, int h, int w, int crop, int ox,
                              int rw, dev_taps ht) {
    const int64_t id = (int64_t) blockIdx.x * blockDim.x + threadIdx.x;
    const int64_t total = (int64_t) n * h * crop;
    if (id >= total) return;
    const int x = (int) (id % crop);
    const int64_t ty = id / crop;                      // t * h + y
    const int sx = x + ox;
    uint8_t * o = mid + id * 3;
    if (sx < 0 || sx >= rw) return;                    // padding column, never read
    const uint8_t * row = src + ty * w * 3;
    if (ht.identity) {
        o[0] = row[sx * 3]; o[1] = row[sx * 3 + 1]; o[2] = row[sx * 3 + 2];
        return;
    }
    const int first = ht.first[sx], cnt = ht.count[sx];
    const int16_t * k = ht.w + (int64_t) sx * ht.ksize;
    const int32_t bias = ht.precision > 0 ? 1 << (ht.precision - 1) : 0;
    int32_t a0 = bias, a1 = bias, a2 = bias;
    const uint8_t * p = row + (int64_t) first * 3;
    for (int j = 0; j < cnt; j++) {
        const int32_t kj = k[j];
        a0 += (int32_t) p[3 * j] * kj;
        a1 += (int32_t) p[3 * j + 1] * kj;
        a2 += (int32_t) p[3 * j + 2] * kj;
    }
    o[0] = clamp_shift(a0, ht.precision);
    o[1] = clamp_shift(a1, ht.precision);
    o[2] = clamp_shift(a2, ht.precision);
}

struct norm_params {
    float mean[3], stdv[3], inv;
    int fused;
};

// out[c][t][y][x] for crop pixel (y, x) of frame t: vertical pass over mid, zero outside the resized
// image, then the normalisation
__global__ void k_resize_cols_norm(const uint8_t * __restrict__ mid, float * __restrict__ out, int n, int h, int crop, int oy, int ox,
                                   int rh, int rw, dev_taps vt, norm_params np) {
    const int64_t id = (int64_t) blockIdx.x * blockDim.x + threadIdx.x;
    const int64_t plane = (int64_t) crop * crop;
    if (id >= (int64_t) n * plane) return;
    const int t = (int) (id / plane);
    const int64_t r = id - (int64_t) t * plane;
    const int y = (int) (r / crop), x = (int) (r - (int64_t) y * crop);
    const int sy = y + oy, sx = x + ox;
    uint8_t v[3] = {0, 0, 0};
    if (sy >= 0 && sy < rh && sx >= 0 && sx < rw) {
        const uint8_t * col = mid + ((int64_t) t * h * crop + x) * 3;   // row y of mid: + y * crop * 3
        if (vt.identity) {
            const uint8_t * p = col + (int64_t) sy * crop * 3;
            v[0] = p[0]; v[1] = p[1]; v[2] = p[2];
        } else {
            const int first = vt.first[sy], cnt = vt.count[sy];
            const int16_t * k = vt.w + (int64_t) sy * vt.ksize;
            const int32_t bias = vt.precision > 0 ? 1 << (vt.precision - 1) : 0;
            int32_t a0 = bias, a1 = bias, a2 = bias;
            for (int j = 0; j < cnt; j++) {
                const uint8_t * p = col + (int64_t) (first + j) * crop * 3;
                const int32_t kj = k[j];
                a0 += (int32_t) p[0] * kj;
                a1 += (int32_t) p[1] * kj;
                a2 += (int32_t) p[2] * kj;
            }
            v[0] = clamp_shift(a0, vt.precision);
            v[1] = clamp_shift(a1, vt.precision);
            v[2] = clamp_shift(a2, vt.precision);
        }
    }
#pragma unroll
    for (int c = 0; c < 3; c++)
        out[((int64_t) c * n + t) * plane + r] = pre_normalize_v(np.fused != 0, np.inv, np.mean[c], np.stdv[c], v[c]);
}

size_t align256(size_t b) { return (b + 255) & ~(size_t) 255; }

size_t taps_bytes(const aa_taps & t) {
    return align256(t.first.size() * 4) + align256(t.count.size() * 4) + align256(t.w.size() * 2);
}

}  // namespace

size_t preprocess_scratch_bytes(const jepa_preprocess_params * p, const pre_plan & g, int n_frames, int h, int w) {
    return taps_bytes(aa_taps_for(w, g.rw, p->resample)) + taps_bytes(aa_taps_for(h, g.rh, p->resample)) +
           align256((size_t) n_frames * h * g.crop * 3);
}

bool launch_preprocess(const jepa_preprocess_params * p, const pre_plan & g, const uint8_t * frames, int n_frames, int h, int w,
                       float * out, void * scratch, hipStream_t s) {
    const aa_taps ht = aa_taps_for(w, g.rw, p->resample), vt = aa_taps_for(h, g.rh, p->resample);
    // table blob: first / count / weights of both passes, 256-byte aligned pieces
    std::vector<unsigned char> blob(taps_bytes(ht) + taps_bytes(vt), 0);
    unsigned char * dev = (unsigned char *) scratch;
    size_t off = 0;
    auto put = [&](const void * src, size_t bytes) -> const void * {
        if (bytes) memcpy(blob.data() + off, src, bytes);
        const void * d = dev + off;
        off += align256(bytes);
        return d;
    };
    dev_taps dh, dv;
    dh.first = (const int *) put(ht.first.data(), ht.first.size() * 4);
    dh.count = (const int *) put(ht.count.data(), ht.count.size() * 4);
    dh.w = (const int16_t *) put(ht.w.data(), ht.w.size() * 2);
    dh.ksize = ht.ksize; dh.precision = ht.precision; dh.identity = g.rw == w;
    dv.first = (const int *) put(vt.first.data(), vt.first.size() * 4);
    dv.count = (const int *) put(vt.count.data(), vt.count.size() * 4);
    dv.w = (const int16_t *) put(vt.w.data(), vt.w.size() * 2);
    dv.ksize = vt.ksize; dv.precision = vt.precision; dv.identity = g.rh == h;
    uint8_t * mid = (uint8_t *) dev + off;
    if (hipMemcpyAsync(scratch, blob.data(), off, hipMemcpyHostToDevice, s) != hipSuccess) return false;
    norm_params np;
    for (int c = 0; c < 3; c++) { np.mean[c] = g.mean[c]; np.stdv[c] = g.stdv[c]; }
    np.inv = g.inv;
    np.fused = g.fused ? 1 : 0;
    const int64_t n1 = (int64_t) n_frames * h * g.crop, n2 = (int64_t) n_frames * g.crop * g.crop;
    k_resize_rows<<<(unsigned) ((n1 + 255) / 256), 256, 0, s>>>(frames, mid, n_frames, h, w, g.crop, g.ox, g.rw, dh);
    k_resize_cols_norm<<<(unsigned) ((n2 + 255) / 256), 256, 0, s>>>(mid, out, n_frames, h, g.crop, g.oy, g.ox, g.rh, g.rw, dv, np);
    // the blob must outlive the copy: wait for it here (pageable source)
    return hipStreamSynchronize(s) == hipSuccess;
}
