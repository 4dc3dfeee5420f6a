// preprocess.hip - uint8 antialiased resize + centre crop + normalisation on the device, equal bit for
// bit to the host jepa_preprocess_frames_rgb_ex (preprocess.cpp; reference src/preprocess.cpp).
//
// The filter tables are built on the host (the double-precision weights and their int16 quantisation
// must be the host's exactly) and uploaded once per call. Two kernels follow the separable order of
// the host resize: the horizontal pass writes only the resized columns the crop keeps, as uint8 (the
// host rounds to uint8 between the passes too); the vertical pass computes the crop's pixels, applies
// the zero padding of an undersized image and writes the normalised floats in NCTHW order.
#include "preprocess.h"
#include "common.h"

#include <cstring>
#include <mutex>

namespace {

// one resample_axis on the device: output o reads inputs lo[o] + t - beg[o] with taps[t],
// beg[o] <= t < beg[o + 1]
struct dev_axis {
    const int32_t * lo;
    const int32_t * beg;
    const int16_t * taps;
    int shift;
    int identity;   // size unchanged: the host skips this pass (a copy)
};

__device__ __forceinline__ uint8_t settle(int32_t acc, int shift) {
    const int32_t v = acc >> shift;
    return (uint8_t) (v < 0 ? 0 : v > 255 ? 255 : v);
}

// mid[t][y][x][c] = horizontal pass of source row y at resized column x + ox, for the crop columns
// that fall inside the resized image
__global__ void k_resize_rows(const uint8_t * __restrict__ src, uint8_t * __restrict__ mid, int n, int h, int w, int crop, int ox,
                              int rw, dev_axis ha) {
    const int64_t id = (int64_t) blockIdx.x * blockDim.x + threadIdx.x;
    const int64_t total = (int64_t) n * h * crop;
    if (id >= total) return;
    const int x = (int) (id % crop);
    const int64_t ty = id / crop;                      // t * h + y
    const int sx = x + ox;
    uint8_t * o = mid + id * 3;
    if (sx < 0 || sx >= rw) return;                    // padding column, never read
    const uint8_t * row = src + ty * w * 3;
    if (ha.identity) {
        o[0] = row[sx * 3]; o[1] = row[sx * 3 + 1]; o[2] = row[sx * 3 + 2];
        return;
    }
    const int32_t half = ha.shift > 0 ? 1 << (ha.shift - 1) : 0;
    int32_t a0 = half, a1 = half, a2 = half;
    const uint8_t * p = row + (int64_t) ha.lo[sx] * 3;
    for (int32_t t = ha.beg[sx], e = ha.beg[sx + 1]; t < e; t++, p += 3) {
        const int32_t k = ha.taps[t];
        a0 += (int32_t) p[0] * k;
        a1 += (int32_t) p[1] * k;
        a2 += (int32_t) p[2] * k;
    }
    o[0] = settle(a0, ha.shift);
    o[1] = settle(a1, ha.shift);
    o[2] = settle(a2, ha.shift);
}

struct norm_params {
    float mean[3], stdv[3], inv;
    int fused;
};

// out[c][t][y][x] for crop pixel (y, x) of frame t: vertical pass over mid, zero outside the resized
// image, then the normalisation
__global__ void k_resize_cols_norm(const uint8_t * __restrict__ mid, float * __restrict__ out, int n, int h, int crop, int oy, int ox,
                                   int rh, int rw, dev_axis va, norm_params np) {
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
        if (va.identity) {
            const uint8_t * p = col + (int64_t) sy * crop * 3;
            v[0] = p[0]; v[1] = p[1]; v[2] = p[2];
        } else {
            const int32_t half = va.shift > 0 ? 1 << (va.shift - 1) : 0;
            int32_t a0 = half, a1 = half, a2 = half;
            const uint8_t * p = col + (int64_t) va.lo[sy] * crop * 3;
            for (int32_t k = va.beg[sy], e = va.beg[sy + 1]; k < e; k++, p += (int64_t) crop * 3) {
                const int32_t tap = va.taps[k];
                a0 += (int32_t) p[0] * tap;
                a1 += (int32_t) p[1] * tap;
                a2 += (int32_t) p[2] * tap;
            }
            v[0] = settle(a0, va.shift);
            v[1] = settle(a1, va.shift);
            v[2] = settle(a2, va.shift);
        }
    }
#pragma unroll
    for (int c = 0; c < 3; c++)
        out[((int64_t) c * n + t) * plane + r] = pre_normalize_v(np.fused != 0, np.inv, np.mean[c], np.stdv[c], v[c]);
}

size_t align256(size_t b) { return (b + 255) & ~(size_t) 255; }

size_t axis_bytes(const resample_axis & ax) {
    return align256(ax.lo.size() * 4) + align256(ax.beg.size() * 4) + align256(ax.taps.size() * 2);
}

}  // namespace

size_t preprocess_scratch_bytes(const jepa_preprocess_params * p, const pre_plan & g, int n_frames, int h, int w) {
    return axis_bytes(resample_axis_for(w, g.rw, p->resample)) + axis_bytes(resample_axis_for(h, g.rh, p->resample)) +
           align256((size_t) n_frames * h * g.crop * 3);
}

namespace {

// Table bytes travel to the device as kernel arguments, PUT_CHUNK bytes per launch: a launch copies
// its arguments when it is enqueued (and a captured launch keeps them in its graph node), so no host
// buffer has to outlive the call, no pinned staging is needed and nothing waits on the stream.
constexpr int PUT_CHUNK = 3072;
struct put_args {
    unsigned char * dst;
    uint32_t n;
    unsigned char b[PUT_CHUNK];
};

__global__ void k_put_bytes(put_args a) {
    for (uint32_t i = threadIdx.x; i < a.n; i += blockDim.x) a.dst[i] = a.b[i];
}

}  // namespace

bool launch_preprocess(const jepa_preprocess_params * p, const pre_plan & g, const uint8_t * frames, int n_frames, int h, int w,
                       float * out, void * scratch, hipStream_t s) {
    const resample_axis hx = resample_axis_for(w, g.rw, p->resample), vx = resample_axis_for(h, g.rh, p->resample);
    // table blob: lo / beg / taps of both passes, 256-byte aligned pieces
    std::vector<unsigned char> blob(axis_bytes(hx) + axis_bytes(vx), 0);
    unsigned char * dev = (unsigned char *) scratch;
    size_t off = 0;
    auto put = [&](const void * src, size_t bytes) -> const void * {
        if (bytes) memcpy(blob.data() + off, src, bytes);
        const void * d = dev + off;
        off += align256(bytes);
        return d;
    };
    auto upload = [&](const resample_axis & ax, bool identity) {
        dev_axis d;
        d.lo = (const int32_t *) put(ax.lo.data(), ax.lo.size() * 4);
        d.beg = (const int32_t *) put(ax.beg.data(), ax.beg.size() * 4);
        d.taps = (const int16_t *) put(ax.taps.data(), ax.taps.size() * 2);
        d.shift = ax.shift;
        d.identity = identity ? 1 : 0;
        return d;
    };
    const dev_axis dh = upload(hx, g.rw == w), dv = upload(vx, g.rh == h);
    uint8_t * mid = (uint8_t *) dev + off;
    for (size_t o = 0; o < off; o += PUT_CHUNK) {
        put_args pa;
        pa.dst = dev + o;
        pa.n = (uint32_t) std::min<size_t>(PUT_CHUNK, off - o);
        memcpy(pa.b, blob.data() + o, pa.n);
        k_put_bytes<<<1, 256, 0, s>>>(pa);
    }
    norm_params np;
    for (int c = 0; c < 3; c++) { np.mean[c] = g.mean[c]; np.stdv[c] = g.stdv[c]; }
    np.inv = g.inv;
    np.fused = g.fused ? 1 : 0;
    const int64_t n1 = (int64_t) n_frames * h * g.crop, n2 = (int64_t) n_frames * g.crop * g.crop;
    k_resize_rows<<<(unsigned) ((n1 + 255) / 256), 256, 0, s>>>(frames, mid, n_frames, h, w, g.crop, g.ox, g.rw, dh);
    k_resize_cols_norm<<<(unsigned) ((n2 + 255) / 256), 256, 0, s>>>(mid, out, n_frames, h, g.crop, g.oy, g.ox, g.rh, g.rw, dv, np);
    return hipGetLastError() == hipSuccess;
}

// ---------------------------------------------------------------------------------------------------
// The same preprocessing without any allocation: the tables and the horizontal-pass image live in a
// file-scope device array. A host reference to `scratch` names a host-side stand-in, not device
// memory; the device address of each GPU's copy comes from hipGetSymbolAddress with that GPU
// current, and only that address is handed to copies and kernels.
// ---------------------------------------------------------------------------------------------------
namespace {
__device__ __align__(256) unsigned char scratch[PRE_NOALLOC_SCRATCH_BYTES];

constexpr int MAX_DEVICES = 64;
std::mutex g_scratch_mu;
void * g_scratch_ptr[MAX_DEVICES] = {};
}  // namespace

void * preprocess_static_scratch(int device) {
    if (device < 0 || device >= MAX_DEVICES) return nullptr;
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    if (!g_scratch_ptr[device]) {
        void * ptr = nullptr;
        const hipError_t e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
        if (e != hipSuccess || !ptr) {
            jepa_log("jepa: hipGetSymbolAddress(scratch) failed on device %d: %s\n", device, hipGetErrorString(e));
            (void) hipGetLastError();
            return nullptr;
        }
        g_scratch_ptr[device] = ptr;
    }
    return g_scratch_ptr[device];
}
