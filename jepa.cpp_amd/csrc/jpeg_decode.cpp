// jpeg_decode.cpp - baseline JPEG (ITU-T T.81 sequential DCT, Huffman, 8-bit) to 8-bit RGB.
//
// Written from the standard: marker syntax (Annex B), Huffman decoding (F.2.2), dequantisation and the
// 8x8 inverse DCT, YCbCr -> RGB by the JFIF equations. The inverse DCT is the Loeffler-Ligtenberg-
// Moschytz factorisation in 13-bit fixed point with 2 extra bits between the passes (the "islow"
// method of the IJG library, its default), and the colour conversion uses 16-bit fixed-point
// coefficients rounded the same way, so that 4:4:4 images decode to the same pixels as libjpeg's
// default settings. Chroma subsampled by 2 is upsampled with the triangle ("fancy") filter; other
// factors are replicated. Progressive, arithmetic-coded, 12-bit and CMYK files are refused.
#include "image_io.h"
#include "model.h"

#include <cstdlib>
#include <cstring>
#include <vector>

namespace {

// zig-zag scan position -> natural (row-major) index of an 8x8 block
const uint8_t kZigzag[64] = {0,  1,  8,  16, 9,  2,  3,  10, 17, 24, 32, 25, 18, 11, 4,  5,  12, 19, 26, 33, 40, 48,
                             41, 34, 27, 20, 13, 6,  7,  14, 21, 28, 35, 42, 49, 56, 57, 50, 43, 36, 29, 22, 15, 23,
                             30, 37, 44, 51, 58, 59, 52, 45, 38, 31, 39, 46, 53, 60, 61, 54, 47, 55, 62, 63};

struct huff {
    // canonical code: codes of length L are mincode[L] .. maxcode[L], values from valptr[L]
    int32_t mincode[17], maxcode[18], valptr[17];
    uint8_t vals[256];
    bool ok = false;
};

bool build_huff(const uint8_t * counts, const uint8_t * vals, int nvals, huff & h) {
    int32_t code = 0, k = 0;
    for (int l = 1; l <= 16; l++) {
        h.valptr[l] = k;
        h.mincode[l] = code;
        code += counts[l - 1];
        k += counts[l - 1];
        h.maxcode[l] = counts[l - 1] ? code - 1 : -1;
        if (code > (1 << l)) return false;
        code <<= 1;
    }
    h.maxcode[17] = 0x7fffffff;
    if (k != nvals || k > 256) return false;
    memcpy(h.vals, vals, (size_t) k);
    h.ok = true;
    return true;
}

struct bit_reader {
    const uint8_t * d;
    size_t n, p;
    uint32_t acc = 0;
    int bits = 0;
    bool marker = false;   // hit a marker: feed zeros
    int fill_byte() {
        if (marker || p >= n) return 0;
        uint8_t b = d[p];
        if (b == 0xff) {
            const uint8_t nx = p + 1 < n ? d[p + 1] : 0;
            if (nx == 0x00) { p += 2; return 0xff; }
            marker = true;
            return 0;
        }
        p++;
        return b;
    }
    int bit() {
        if (bits == 0) { acc = (uint32_t) fill_byte(); bits = 8; }
        bits--;
        return (int) ((acc >> bits) & 1);
    }
    int get(int k) {
        int v = 0;
        for (int i = 0; i < k; i++) v = (v << 1) | bit();
        return v;
    }
    void reset() { bits = 0; acc = 0; }
};

int decode_sym(bit_reader & br, const huff & h) {
    int32_t code = br.bit();
    int l = 1;
    while (l <= 16 && code > h.maxcode[l]) { code = (code << 1) | br.bit(); l++; }
    if (l > 16) return -1;
    return h.vals[h.valptr[l] + code - h.mincode[l]];
}

int extend(int v, int t) { return t == 0 ? 0 : v < (1 << (t - 1)) ? v - (1 << t) + 1 : v; }

// islow inverse DCT of one dequantised block (natural order) into 8x8 samples with the 128 level shift
constexpr int CB = 13, P1 = 2;
constexpr int32_t F0298 = 2446, F0390 = 3196, F0541 = 4433, F0765 = 6270, F0899 = 7373, F1175 = 9633, F1501 = 12299,
                  F1847 = 15137, F1961 = 16069, F2053 = 16819, F2562 = 20995, F3072 = 25172;
inline int32_t descale(int64_t x, int n) { return (int32_t) ((x + ((int64_t) 1 << (n - 1))) >> n); }
inline uint8_t clamp8(int v) { return (uint8_t) (v < 0 ? 0 : v > 255 ? 255 : v); }

template <bool ROWS>
void idct_1d(const int32_t * in, int stride_in, int32_t * out, int stride_out, uint8_t * o8) {
    constexpr int SH = ROWS ? CB + P1 + 3 : CB - P1;
    const int64_t s0 = in[0], s1 = in[stride_in], s2 = in[2 * stride_in], s3 = in[3 * stride_in], s4 = in[4 * stride_in],
                  s5 = in[5 * stride_in], s6 = in[6 * stride_in], s7 = in[7 * stride_in];
    int32_t r[8];
    if (!s1 && !s2 && !s3 && !s4 && !s5 && !s6 && !s7) {
        const int32_t dc = ROWS ? descale(s0, P1 + 3) : (int32_t) (s0 * (1 << P1));
        for (int i = 0; i < 8; i++) r[i] = dc;
    } else {
        // even part
        int64_t z1 = (s2 + s6) * F0541;
        const int64_t t2 = z1 - s6 * F1847, t3 = z1 + s2 * F0765;
        const int64_t t0 = (s0 + s4) * (1 << CB), t1 = (s0 - s4) * (1 << CB);
        const int64_t t10 = t0 + t3, t13 = t0 - t3, t11 = t1 + t2, t12 = t1 - t2;
        // odd part
        int64_t o0 = s7, o1 = s5, o2 = s3, o3 = s1;
        int64_t a1 = o0 + o3, a2 = o1 + o2, a3 = o0 + o2, a4 = o1 + o3;
        const int64_t z5 = (a3 + a4) * F1175;
        o0 *= F0298; o1 *= F2053; o2 *= F3072; o3 *= F1501;
        a1 *= -F0899; a2 *= -F2562; a3 *= -F1961; a4 *= -F0390;
        a3 += z5; a4 += z5;
        o0 += a1 + a3; o1 += a2 + a4; o2 += a2 + a3; o3 += a1 + a4;
        r[0] = descale(t10 + o3, SH); r[7] = descale(t10 - o3, SH);
        r[1] = descale(t11 + o2, SH); r[6] = descale(t11 - o2, SH);
        r[2] = descale(t12 + o1, SH); r[5] = descale(t12 - o1, SH);
        r[3] = descale(t13 + o0, SH); r[4] = descale(t13 - o0, SH);
    }
    for (int i = 0; i < 8; i++) {
        if (ROWS) o8[i] = clamp8(r[i] + 128);
        else out[i * stride_out] = r[i];
    }
}

void idct8x8(const int32_t * coef, uint8_t * dst, int stride) {
    int32_t ws[64];
    for (int c = 0; c < 8; c++) idct_1d<false>(coef + c, 8, ws + c, 8, nullptr);
    for (int r = 0; r < 8; r++) idct_1d<true>(ws + r * 8, 1, nullptr, 0, dst + (size_t) r * stride);
}

struct comp {
    int id, h, v, tq;
    int td = 0, ta = 0;
    int pred = 0;
    int bw = 0, bh = 0;               // blocks per row / column (padded to whole MCUs)
    std::vector<uint8_t> pix;         // bw*8 x bh*8 samples
};

// JFIF YCbCr -> RGB in 16-bit fixed point, each product rounded as the tables of libjpeg's default
// converter are (R and B add a rounded product, G rounds the sum of two products)
struct ycc_tables {
    int cr_r[256], cb_b[256], cr_g[256], cb_g[256];
    ycc_tables() {
        const int64_t ONE_HALF = 1 << 15;
        auto fix = [](double x) { return (int64_t) (x * 65536.0 + 0.5); };
        for (int i = 0; i < 256; i++) {
            const int64_t x = i - 128;
            cr_r[i] = (int) ((fix(1.40200) * x + ONE_HALF) >> 16);
            cb_b[i] = (int) ((fix(1.77200) * x + ONE_HALF) >> 16);
            cr_g[i] = (int) (-fix(0.71414) * x);
            cb_g[i] = (int) (-fix(0.34414) * x + ONE_HALF);
        }
    }
};

// one upsampled output row of a component subsampled by 2 horizontally (and vertically when v2):
// the triangle filter weights 3/4 : 1/4 of the nearer and farther input sample
void upsample_row(const comp & c, int y_out, int W, int Hc, int hs, int vs, std::vector<uint8_t> & row) {
    const int stride = c.bw * 8;
    row.resize((size_t) W);
    if (vs == 2 && hs == 2 && c.h == 1 && c.v == 1) {
        const int yi = y_out / 2;
        const int yn = (y_out & 1) ? (yi + 1 < Hc ? yi + 1 : yi) : (yi > 0 ? yi - 1 : 0);   // the farther row
        const uint8_t * a = c.pix.data() + (size_t) yi * stride;
        const uint8_t * b = c.pix.data() + (size_t) yn * stride;
        const int Wc = (W + 1) / 2;
        std::vector<int> col((size_t) Wc);
        for (int x = 0; x < Wc; x++) col[(size_t) x] = 3 * a[x] + b[x];
        if (Wc == 1) { row[0] = (uint8_t) ((col[0] * 4 + 8) >> 4); if (W > 1) row[1] = row[0]; return; }
        for (int x = 0; x < Wc; x++) {
            const int cur = col[(size_t) x];
            const int left = col[(size_t) (x > 0 ? x - 1 : 0)], right = col[(size_t) (x + 1 < Wc ? x + 1 : Wc - 1)];
            const int o0 = x == 0 ? (cur * 4 + 8) >> 4 : (cur * 3 + left + 8) >> 4;
            const int o1 = x == Wc - 1 ? (cur * 4 + 7) >> 4 : (cur * 3 + right + 7) >> 4;
            if (2 * x < W) row[(size_t) (2 * x)] = (uint8_t) o0;
            if (2 * x + 1 < W) row[(size_t) (2 * x + 1)] = (uint8_t) o1;
        }
        return;
    }
    const int yi = y_out * c.v / vs;
    const uint8_t * a = c.pix.data() + (size_t) yi * stride;
    if (hs == 2 && c.h == 1) {
        const int Wc = (W + 1) / 2;
        for (int x = 0; x < Wc; x++) {
            const int cur = a[x], left = a[x > 0 ? x - 1 : 0], right = a[x + 1 < Wc ? x + 1 : Wc - 1];
            const int o0 = x == 0 ? cur : (cur * 3 + left + 1) >> 2;
            const int o1 = x == Wc - 1 ? cur : (cur * 3 + right + 2) >> 2;
            if (2 * x < W) row[(size_t) (2 * x)] = (uint8_t) o0;
            if (2 * x + 1 < W) row[(size_t) (2 * x + 1)] = (uint8_t) o1;
        }
        return;
    }
    for (int x = 0; x < W; x++) row[(size_t) x] = a[x * c.h / hs];
}

}  // namespace

uint8_t * decode_jpeg(const uint8_t * d, size_t n, int * ph, int * pw, const char * path) {
    auto fail = [&](const char * why) -> uint8_t * {
        jepa_log("jepa: cannot decode image %s: %s\n", path, why);
        return nullptr;
    };
    int32_t qt[4][64];
    bool qok[4] = {false, false, false, false};
    huff hdc[4], hac[4];
    std::vector<comp> comps;
    int W = 0, H = 0, restart = 0, hmax = 1, vmax = 1;
    bool adobe_rgb = false;
    size_t p = 2;
    while (p + 4 <= n) {
        if (d[p] != 0xff) { p++; continue; }
        const uint8_t m = d[p + 1];
        if (m == 0xff) { p++; continue; }
        if (m == 0xd8 || (m >= 0xd0 && m <= 0xd7) || m == 0x01) { p += 2; continue; }
        if (m == 0xd9) break;
        const size_t len = (size_t) d[p + 2] << 8 | d[p + 3];
        if (len < 2 || p + 2 + len > n) return fail("truncated JPEG segment");
        const uint8_t * s = d + p + 4;
        const size_t sl = len - 2;
        if (m == 0xdb) {                                  // DQT
            size_t q = 0;
            while (q < sl) {
                const int pq = s[q] >> 4, tq = s[q] & 15;
                if (tq > 3 || q + 1 + 64 * (pq ? 2 : 1) > sl) return fail("bad quantisation table");
                for (int i = 0; i < 64; i++)
                    qt[tq][kZigzag[i]] = pq ? (s[q + 1 + 2 * i] << 8 | s[q + 2 + 2 * i]) : s[q + 1 + i];
                qok[tq] = true;
                q += 1 + 64 * (pq ? 2 : 1);
            }
        } else if (m == 0xc4) {                           // DHT
            size_t q = 0;
            while (q + 17 <= sl) {
                const int tc = s[q] >> 4, th = s[q] & 15;
                int nv = 0;
                for (int i = 0; i < 16; i++) nv += s[q + 1 + i];
                if (th > 3 || tc > 1 || q + 17 + nv > sl) return fail("bad Huffman table");
                if (!build_huff(s + q + 1, s + q + 17, nv, tc ? hac[th] : hdc[th])) return fail("bad Huffman table");
                q += 17 + nv;
            }
        } else if (m == 0xdd) {                           // DRI
            if (sl < 2) return fail("bad restart interval");
            restart = s[0] << 8 | s[1];
        } else if (m == 0xee && sl >= 12 && !memcmp(s, "Adobe", 5)) {
            adobe_rgb = s[11] == 0;                        // transform 0: components are RGB (or CMYK)
        } else if (m == 0xc0 || m == 0xc1) {              // SOF0 / SOF1
            if (sl < 6 || s[0] != 8) return fail("only 8-bit JPEG is supported");
            H = s[1] << 8 | s[2];
            W = s[3] << 8 | s[4];
            const int nc = s[5];
            if (W <= 0 || H <= 0 || (nc != 1 && nc != 3) || sl < (size_t) (6 + 3 * nc) || (int64_t) W * H > (1ll << 28))
                return fail("unsupported JPEG frame");
            for (int i = 0; i < nc; i++) {
                comp c;
                c.id = s[6 + 3 * i]; c.h = s[7 + 3 * i] >> 4; c.v = s[7 + 3 * i] & 15; c.tq = s[8 + 3 * i];
                if (c.h < 1 || c.h > 2 || c.v < 1 || c.v > 2 || c.tq > 3) return fail("unsupported JPEG sampling");
                hmax = c.h > hmax ? c.h : hmax;
                vmax = c.v > vmax ? c.v : vmax;
                comps.push_back(c);
            }
        } else if ((m >= 0xc2 && m <= 0xcf) && m != 0xc4 && m != 0xc8 && m != 0xcc) {
            return fail("progressive, lossless or arithmetic-coded JPEG is not supported");
        } else if (m == 0xda) {                           // SOS: one interleaved scan of every component
            if (comps.empty() || sl < 1) return fail("scan before frame header");
            const int ns = s[0];
            if (ns != (int) comps.size() || sl < (size_t) (1 + 2 * ns + 3)) return fail("only single-scan baseline JPEG is supported");
            for (int i = 0; i < ns; i++) {
                const int cid = s[1 + 2 * i];
                bool found = false;
                for (auto & c : comps)
                    if (c.id == cid) { c.td = s[2 + 2 * i] >> 4; c.ta = s[2 + 2 * i] & 15; found = true; }
                if (!found) return fail("scan names an unknown component");
            }
            for (auto & c : comps)
                if (c.td > 3 || c.ta > 3 || !hdc[c.td].ok || !hac[c.ta].ok || !qok[c.tq]) return fail("missing JPEG table");
            const int mcux = (W + 8 * hmax - 1) / (8 * hmax), mcuy = (H + 8 * vmax - 1) / (8 * vmax);
            for (auto & c : comps) {
                c.bw = mcux * c.h; c.bh = mcuy * c.v;
                c.pix.assign((size_t) c.bw * 8 * c.bh * 8, 0);
                c.pred = 0;
            }
            bit_reader br{d, n, p + 2 + len};
            int32_t blk[64];
            int todo = restart;
            for (int my = 0; my < mcuy; my++)
                for (int mx = 0; mx < mcux; mx++) {
                    if (restart && todo == 0) {   // RSTn: byte-align, skip the marker, reset predictions
                        br.reset();
                        while (br.p + 1 < n && !(br.d[br.p] == 0xff && br.d[br.p + 1] >= 0xd0 && br.d[br.p + 1] <= 0xd7)) br.p++;
                        if (br.p + 1 < n) br.p += 2;
                        br.marker = false;
                        for (auto & c : comps) c.pred = 0;
                        todo = restart;
                    }
                    for (auto & c : comps)
                        for (int by = 0; by < c.v; by++)
                            for (int bx = 0; bx < c.h; bx++) {
                                memset(blk, 0, sizeof(blk));
                                const int t = decode_sym(br, hdc[c.td]);
                                if (t < 0 || t > 11) return fail("corrupt JPEG data");
                                c.pred += extend(br.get(t), t);
                                blk[0] = c.pred * qt[c.tq][0];
                                for (int k = 1; k < 64;) {
                                    const int rs = decode_sym(br, hac[c.ta]);
                                    if (rs < 0) return fail("corrupt JPEG data");
                                    const int r = rs >> 4, sz = rs & 15;
                                    if (sz == 0) {
                                        if (r != 15) break;   // end of block
                                        k += 16;
                                        continue;
                                    }
                                    k += r;
                                    if (k > 63) return fail("corrupt JPEG data");
                                    const int z = kZigzag[k];
                                    blk[z] = extend(br.get(sz), sz) * qt[c.tq][z];
                                    k++;
                                }
                                const int bxx = mx * c.h + bx, byy = my * c.v + by;
                                idct8x8(blk, c.pix.data() + ((size_t) byy * 8 * c.bw * 8 + (size_t) bxx * 8), c.bw * 8);
                            }
                    if (restart) todo--;
                }
            // colour conversion (and chroma upsampling) into RGB
            uint8_t * out = (uint8_t *) malloc((size_t) W * H * 3);
            if (!out) return nullptr;
            static const ycc_tables tab;
            std::vector<uint8_t> r0, r1, r2;
            for (int y = 0; y < H; y++) {
                const uint8_t * yr;
                if (comps[0].h != hmax || comps[0].v != vmax) {
                    upsample_row(comps[0], y, W, (H * comps[0].v + vmax - 1) / vmax, hmax, vmax, r0);
                    yr = r0.data();
                } else {
                    yr = comps[0].pix.data() + (size_t) y * comps[0].bw * 8;
                }
                uint8_t * o = out + (size_t) y * W * 3;
                if (comps.size() == 1) {
                    for (int x = 0; x < W; x++) o[3 * x] = o[3 * x + 1] = o[3 * x + 2] = yr[x];
                    continue;
                }
                const uint8_t * cb;
                const uint8_t * cr;
                if (comps[1].h == hmax && comps[1].v == vmax) cb = comps[1].pix.data() + (size_t) y * comps[1].bw * 8;
                else { upsample_row(comps[1], y, W, (H * comps[1].v + vmax - 1) / vmax, hmax, vmax, r1); cb = r1.data(); }
                if (comps[2].h == hmax && comps[2].v == vmax) cr = comps[2].pix.data() + (size_t) y * comps[2].bw * 8;
                else { upsample_row(comps[2], y, W, (H * comps[2].v + vmax - 1) / vmax, hmax, vmax, r2); cr = r2.data(); }
                for (int x = 0; x < W; x++) {
                    if (adobe_rgb) { o[3 * x] = yr[x]; o[3 * x + 1] = cb[x]; o[3 * x + 2] = cr[x]; continue; }
                    const int Y = yr[x], B = cb[x], R = cr[x];
                    o[3 * x] = clamp8(Y + tab.cr_r[R]);
                    o[3 * x + 1] = clamp8(Y + ((tab.cb_g[B] + tab.cr_g[R]) >> 16));
                    o[3 * x + 2] = clamp8(Y + tab.cb_b[B]);
                }
            }
            *ph = H;
            *pw = W;
            return out;
        }
        p += 2 + len;
    }
    return fail("no baseline JPEG scan found");
}
