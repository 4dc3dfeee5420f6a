// image_io.cpp - jepa_load_image_rgb: image files to 8-bit RGB HWC (reference src/preprocess.cpp:183-193,
// which decodes with stb_image). Formats decoded here, by this file's own readers:
//   - PNG (8- and 16-bit; grey, grey+alpha, RGB, RGBA, palette; non-interlaced and Adam7), the zlib
//     stream inflated by the system zlib;
//   - binary PPM / PGM (P6 / P5, maxval <= 255);
//   - JPEG (jpeg_decode.cpp).
// Alpha is dropped (not composited) and grey is replicated, as stb_image does when asked for three
// channels; 16-bit samples keep their high byte.
#include "image_io.h"
#include "model.h"

#include <zlib.h>

#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <vector>

namespace {

constexpr int64_t MAX_PIXELS = 1ll << 28;   // 16384 x 16384 (products of header sizes are formed only where they cannot overflow)

bool read_file(const char * path, std::vector<uint8_t> & buf) {
    FILE * f = fopen(path, "rb");
    if (!f) return false;
    bool ok = fseek(f, 0, SEEK_END) == 0;
    const long n = ok ? ftell(f) : -1;
    ok = ok && n >= 0 && fseek(f, 0, SEEK_SET) == 0;
    if (ok) {
        buf.resize((size_t) n);
        ok = n == 0 || fread(buf.data(), 1, (size_t) n, f) == (size_t) n;
    }
    fclose(f);
    return ok;
}

uint32_t be32(const uint8_t * p) { return (uint32_t) p[0] << 24 | (uint32_t) p[1] << 16 | (uint32_t) p[2] << 8 | p[3]; }

uint8_t paeth(int a, int b, int c) {
    const int p = a + b - c, pa = abs(p - a), pb = abs(p - b), pc = abs(p - c);
    return (uint8_t) (pa <= pb && pa <= pc ? a : pb <= pc ? b : c);
}

// undo the PNG row filters of a (sub)image of w x h pixels, bpp bytes per pixel (>= 1), rowbytes per
// row, in place on `data` laid out as h rows of (1 filter byte + rowbytes)
bool unfilter(uint8_t * data, int64_t w, int64_t h, int bpp, int64_t rowbytes, std::vector<uint8_t> & out) {
    out.assign((size_t) (rowbytes * h), 0);
    (void) w;
    for (int64_t y = 0; y < h; y++) {
        const uint8_t ft = data[y * (rowbytes + 1)];
        const uint8_t * in = data + y * (rowbytes + 1) + 1;
        uint8_t * cur = out.data() + y * rowbytes;
        const uint8_t * prev = y > 0 ? cur - rowbytes : nullptr;
        for (int64_t i = 0; i < rowbytes; i++) {
            const int a = i >= bpp ? cur[i - bpp] : 0, b = prev ? prev[i] : 0, c = (prev && i >= bpp) ? prev[i - bpp] : 0;
            int v = in[i];
            switch (ft) {
                case 0: break;
                case 1: v += a; break;
                case 2: v += b; break;
                case 3: v += (a + b) >> 1; break;
                case 4: v += paeth(a, b, c); break;
                default: return false;
            }
            cur[i] = (uint8_t) v;
        }
    }
    return true;
}

uint8_t * decode_png(const std::vector<uint8_t> & f, int * ph, int * pw, const char * path) {
    size_t p = 8;
    uint32_t W = 0, H = 0;
    int depth = 0, ctype = -1, interlace = 0;
    std::vector<uint8_t> idat, plte;
    bool ihdr = false, iend = false;
    while (p + 12 <= f.size() && !iend) {
        const uint32_t len = be32(&f[p]);
        const uint8_t * type = &f[p + 4];
        if (len > f.size() - p - 12) break;
        const uint8_t * d = &f[p + 8];
        if (!memcmp(type, "IHDR", 4) && len >= 13) {
            W = be32(d); H = be32(d + 4); depth = d[8]; ctype = d[9]; interlace = d[12];
            ihdr = true;
        } else if (!memcmp(type, "PLTE", 4)) {
            plte.assign(d, d + len);
        } else if (!memcmp(type, "IDAT", 4)) {
            idat.insert(idat.end(), d, d + len);
        } else if (!memcmp(type, "IEND", 4)) {
            iend = true;
        }
        p += 12 + (size_t) len;
    }
    const int chans = ctype == 0 ? 1 : ctype == 2 ? 3 : ctype == 3 ? 1 : ctype == 4 ? 2 : ctype == 6 ? 4 : 0;
    if (!ihdr || W == 0 || H == 0 || chans == 0 || interlace > 1 || (uint64_t) W * H > (uint64_t) MAX_PIXELS ||
        !(depth == 8 || depth == 16 || (depth < 8 && (ctype == 0 || ctype == 3) && (depth == 1 || depth == 2 || depth == 4))) ||
        (ctype == 3 && (plte.size() < 3 || depth == 16))) {
        jepa_log("jepa: cannot decode image %s: unsupported or corrupt PNG\n", path);
        return nullptr;
    }
    const int bits = chans * depth;                 // per pixel
    const int bpp = bits >= 8 ? bits / 8 : 1;       // filter distance in bytes
    // passes: one full image, or the 7 Adam7 sub-images
    static const int ax0[7] = {0, 4, 0, 2, 0, 1, 0}, ay0[7] = {0, 0, 4, 0, 2, 0, 1}, adx[7] = {8, 8, 4, 4, 2, 2, 1},
                     ady[7] = {8, 8, 8, 4, 4, 2, 2};
    const int npass = interlace ? 7 : 1;
    size_t raw_size = 0;
    for (int k = 0; k < npass; k++) {
        const int64_t pw = interlace ? ((int64_t) W - ax0[k] + adx[k] - 1) / adx[k] : W;
        const int64_t phh = interlace ? ((int64_t) H - ay0[k] + ady[k] - 1) / ady[k] : H;
        if (pw > 0 && phh > 0) raw_size += (size_t) ((pw * bits + 7) / 8 + 1) * phh;
    }
    std::vector<uint8_t> raw(raw_size);
    uLongf got = (uLongf) raw_size;
    if (uncompress(raw.data(), &got, idat.data(), (uLong) idat.size()) != Z_OK || got != raw_size) {
        jepa_log("jepa: cannot decode image %s: corrupt PNG data\n", path);
        return nullptr;
    }
    uint8_t * out = (uint8_t *) malloc((size_t) W * H * 3);
    if (!out) return nullptr;
    std::vector<uint8_t> px;
    size_t off = 0;
    for (int k = 0; k < npass; k++) {
        const int64_t pw = interlace ? ((int64_t) W - ax0[k] + adx[k] - 1) / adx[k] : W;
        const int64_t phh = interlace ? ((int64_t) H - ay0[k] + ady[k] - 1) / ady[k] : H;
        if (pw <= 0 || phh <= 0) continue;
        const int64_t rowbytes = (pw * bits + 7) / 8;
        if (!unfilter(raw.data() + off, pw, phh, bpp, rowbytes, px)) {
            free(out);
            jepa_log("jepa: cannot decode image %s: bad PNG filter\n", path);
            return nullptr;
        }
        off += (size_t) (rowbytes + 1) * phh;
        for (int64_t y = 0; y < phh; y++) {
            const uint8_t * row = px.data() + y * rowbytes;
            for (int64_t x = 0; x < pw; x++) {
                int s[4] = {0, 0, 0, 0};
                for (int c = 0; c < chans; c++) {
                    if (depth == 8) s[c] = row[x * chans + c];
                    else if (depth == 16) s[c] = row[(x * chans + c) * 2];   // high byte
                    else {
                        const int64_t bit = x * depth;
                        const int v = (row[bit >> 3] >> (8 - depth - (int) (bit & 7))) & ((1 << depth) - 1);
                        s[c] = ctype == 3 ? v : v * (255 / ((1 << depth) - 1));   // grey scaled to 0..255
                    }
                }
                uint8_t rgb[3];
                if (ctype == 3) {
                    const size_t i = (size_t) s[0] * 3;
                    if (i + 2 >= plte.size()) rgb[0] = rgb[1] = rgb[2] = 0;
                    else { rgb[0] = plte[i]; rgb[1] = plte[i + 1]; rgb[2] = plte[i + 2]; }
                } else if (chans <= 2) {
                    rgb[0] = rgb[1] = rgb[2] = (uint8_t) s[0];
                } else {
                    rgb[0] = (uint8_t) s[0]; rgb[1] = (uint8_t) s[1]; rgb[2] = (uint8_t) s[2];
                }
                const int64_t X = interlace ? ax0[k] + x * adx[k] : x, Y = interlace ? ay0[k] + y * ady[k] : y;
                memcpy(out + ((size_t) Y * W + X) * 3, rgb, 3);
            }
        }
    }
    *ph = (int) H;
    *pw = (int) W;
    return out;
}

// P5 / P6 with one whitespace-separated header (comments allowed), maxval <= 255
uint8_t * decode_pnm(const std::vector<uint8_t> & f, int * ph, int * pw, const char * path) {
    size_t p = 2;
    auto num = [&](long & v) {
        for (;;) {
            while (p < f.size() && isspace(f[p])) p++;
            if (p < f.size() && f[p] == '#') { while (p < f.size() && f[p] != '\n') p++; continue; }
            break;
        }
        if (p >= f.size() || !isdigit(f[p])) return false;
        v = 0;
        while (p < f.size() && isdigit(f[p]) && v < (1l << 30)) v = v * 10 + (f[p++] - '0');
        return true;
    };
    long W = 0, H = 0, mx = 0;
    const int chans = f[1] == '6' ? 3 : 1;
    if (!num(W) || !num(H) || !num(mx) || p >= f.size() || W <= 0 || H <= 0 || mx <= 0 || mx > 255 || W > MAX_PIXELS || H > MAX_PIXELS ||
        (int64_t) W * H > MAX_PIXELS ||
        f.size() - p - 1 < (size_t) W * H * chans) {
        jepa_log("jepa: cannot decode image %s: unsupported or truncated PNM\n", path);
        return nullptr;
    }
    p++;   // the single whitespace after maxval
    uint8_t * out = (uint8_t *) malloc((size_t) W * H * 3);
    if (!out) return nullptr;
    for (int64_t i = 0; i < (int64_t) W * H; i++)
        for (int c = 0; c < 3; c++) out[i * 3 + c] = f[p + (size_t) i * chans + (chans == 3 ? c : 0)];
    *ph = (int) H;
    *pw = (int) W;
    return out;
}

}  // namespace

extern "C" uint8_t * jepa_load_image_rgb(const char * path, int * h, int * w) {
    if (!path || !h || !w) return nullptr;
    std::vector<uint8_t> f;
    if (!read_file(path, f)) {
        jepa_log("jepa: cannot decode image %s: cannot read the file\n", path);
        return nullptr;
    }
    static const uint8_t png_sig[8] = {0x89, 'P', 'N', 'G', 0x0d, 0x0a, 0x1a, 0x0a};
    if (f.size() >= 8 && !memcmp(f.data(), png_sig, 8)) return decode_png(f, h, w, path);
    if (f.size() >= 2 && f[0] == 0xff && f[1] == 0xd8) return decode_jpeg(f.data(), f.size(), h, w, path);
    if (f.size() >= 3 && f[0] == 'P' && (f[1] == '5' || f[1] == '6')) return decode_pnm(f, h, w, path);
    jepa_log("jepa: cannot decode image %s: not a PNG, JPEG or binary PPM/PGM file\n", path);
    return nullptr;
}
