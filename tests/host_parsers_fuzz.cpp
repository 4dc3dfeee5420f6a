// host_parsers_fuzz.cpp - seeded mutation campaign over the library's host-side parsers of untrusted
// files, built by tests/test_host_parsers_asan.py with AddressSanitizer and UndefinedBehaviorSanitizer
// (host code only, no GPU): every out-of-bounds access, use after free, leak, overflow or other
// undefined behaviour aborts the run.
//
//   host_parsers_fuzz image <seed file> <scratch path> <iterations> <rng seed>
//       mutates the seed (JPEG / PNG / PPM), writes it to the scratch path and loads it with
//       jepa_load_image_rgb (image_io.cpp, jpeg_decode.cpp); a decoded image is read whole and run
//       through jepa_preprocess_image_rgb_ex (preprocess.cpp) and jepa_resize_antialias_u8.
//   host_parsers_fuzz gguf <seed file> <scratch path> <iterations> <rng seed>
//       mutates the header, metadata and tensor-info bytes of a GGUF file (before its data section)
//       and parses it with gguf::open (gguf.cpp), rendering every value of an accepted file.
//
//   host_parsers_fuzz image-check|gguf-check <file> - 0 0
//       loads one file as it is (hostile headers kept as regression cases).
//
// Prints "ok <accepted> refused <rejected>" and exits 0 when no sanitizer fired.
#include "gguf.h"
#include "image_io.h"
#include "jepa.h"

#include <algorithm>
#include <cstdarg>
#include <cstdint>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <string>
#include <vector>

// the library's logger, jepa_free (= free, include/jepa.h) and model defaults live in api.cpp, which
// needs the HIP runtime; the parsers only log refusals and the preprocessing here takes explicit
// parameters
void jepa_log(const char * fmt, ...) {
    (void) fmt;
}
extern "C" void jepa_free(void * p) { free(p); }
extern "C" jepa_preprocess_params jepa_preprocess_default_params(const jepa_model *) {
    jepa_preprocess_params p;
    const float mean[3] = {0.485f, 0.456f, 0.406f}, sd[3] = {0.229f, 0.224f, 0.225f};
    for (int i = 0; i < 3; i++) { p.mean[i] = mean[i]; p.std[i] = sd[i]; }
    p.resize_short = 256; p.crop = 224;
    p.resample = JEPA_RESAMPLE_BILINEAR; p.resize_mode = JEPA_RESIZE_SHORTEST_EDGE;
    p.rescale = 1.0f / 255.0f; p.fused_norm = true;
    return p;
}

namespace {

struct rng {
    uint64_t s;
    explicit rng(uint64_t seed) : s(seed ? seed : 0x9E3779B97F4A7C15ull) {}
    uint64_t next() {   // xorshift64*
        s ^= s >> 12; s ^= s << 25; s ^= s >> 27;
        return s * 0x2545F4914F6CDD1Dull;
    }
    size_t below(size_t n) { return n ? (size_t) (next() % n) : 0; }
};

bool read_all(const char * path, std::vector<uint8_t> & out) {
    FILE * f = fopen(path, "rb");
    if (!f) return false;
    uint8_t buf[65536];
    size_t n;
    while ((n = fread(buf, 1, sizeof buf, f)) > 0) out.insert(out.end(), buf, buf + n);
    fclose(f);
    return true;
}

bool write_all(const char * path, const std::vector<uint8_t> & d) {
    FILE * f = fopen(path, "wb");
    if (!f) return false;
    const bool ok = d.empty() || fwrite(d.data(), 1, d.size(), f) == d.size();
    return fclose(f) == 0 && ok;
}

// One to four edits, each at an offset below `hot` half of the time (the headers) and anywhere
// below `limit` otherwise.
void mutate(std::vector<uint8_t> & d, rng & r, size_t hot, size_t limit) {
    const int n = 1 + (int) r.below(4);
    for (int k = 0; k < n && !d.empty(); k++) {
        const size_t lim = std::min(limit, d.size());
        const size_t off = r.below(2) ? r.below(std::min(hot, lim)) : r.below(lim);
        switch (r.below(6)) {
            case 0: d[off] ^= (uint8_t) (1u << r.below(8)); break;
            case 1: {
                static const uint8_t v[] = {0x00, 0xFF, 0x7F, 0x80, 0x01, 0xFE};
                d[off] = v[r.below(sizeof v)];
                break;
            }
            case 2: {   // a 32-bit field, either byte order (PNG and JPEG are big-endian, GGUF little)
                const uint32_t v[] = {0u, 1u, 0xFFFFFFFFu, 0x7FFFFFFFu, 0x80000000u, 0xFFFFu, 0x10000u,
                                      (uint32_t) d.size(), (uint32_t) d.size() + 1u, (uint32_t) r.next()};
                const uint32_t x = v[r.below(sizeof v / sizeof v[0])];
                const bool be = r.below(2);
                for (int b = 0; b < 4 && off + b < d.size(); b++) d[off + b] = (uint8_t) (x >> (8 * (be ? 3 - b : b)));
                break;
            }
            case 3: {   // a 64-bit little-endian count or length
                const uint64_t v[] = {0ull, 1ull, ~0ull, 1ull << 63, 1ull << 32, (uint64_t) d.size(), 0x7FFFFFFFFFFFFFFFull,
                                      r.next()};
                const uint64_t x = v[r.below(sizeof v / sizeof v[0])];
                for (int b = 0; b < 8 && off + b < d.size(); b++) d[off + b] = (uint8_t) (x >> (8 * b));
                break;
            }
            case 4: d.resize(off); break;
            case 5: {   // copy a chunk of up to 64 bytes over another place
                const size_t src = r.below(d.size()), len = 1 + r.below(64);
                for (size_t i = 0; i < len && src + i < d.size() && off + i < d.size(); i++) d[off + i] = d[src + i];
                break;
            }
        }
    }
}

uint64_t touch(const uint8_t * p, size_t n) {   // reads every byte (the sanitizer sees each access)
    uint64_t h = 1469598103934665603ull;
    for (size_t i = 0; i < n; i++) h = (h ^ p[i]) * 1099511628211ull;
    return h;
}

bool run_image(const char * scratch, uint64_t & sink) {
    int h = 0, w = 0;
    uint8_t * rgb = jepa_load_image_rgb(scratch, &h, &w);
    if (!rgb) return false;
    if (h <= 0 || w <= 0) { fprintf(stderr, "decoder returned an image of %d x %d\n", h, w); abort(); }
    sink ^= touch(rgb, (size_t) h * w * 3);
    if ((int64_t) h * w <= (int64_t) 4096 * 4096) {
        jepa_preprocess_params p = jepa_preprocess_default_params(nullptr);
        for (int v = 0; v < 2; v++) {
            if (v == 1) { p.resample = JEPA_RESAMPLE_BICUBIC; p.resize_mode = JEPA_RESIZE_SQUASH; p.crop = 64; p.resize_short = 64; }
            int oh = 0, ow = 0;
            float * x = jepa_preprocess_image_rgb_ex(&p, rgb, h, w, &oh, &ow);
            if (x) { sink ^= touch((const uint8_t *) x, (size_t) 3 * oh * ow * sizeof(float)); jepa_free(x); }
        }
        std::vector<uint8_t> small((size_t) 17 * 29 * 3);
        jepa_resize_antialias_u8(rgb, h, w, 3, small.data(), 17, 29, 1);
        sink ^= touch(small.data(), small.size());
    }
    jepa_free(rgb);
    return true;
}

bool run_gguf(const char * scratch, uint64_t & sink) {
    gguf::file f;
    std::string err;
    if (!gguf::open(scratch, f, err)) return false;
    for (const auto & kv : f.kv) sink ^= touch((const uint8_t *) kv.second.render().data(), kv.second.render().size());
    for (const auto & t : f.tensors) sink ^= t.nbytes + t.offset + (uint64_t) t.n_dims;
    return true;
}

}  // namespace

int main(int argc, char ** argv) {
    if (argc != 6) {
        fprintf(stderr, "usage: %s image|gguf <seed file> <scratch path> <iterations> <rng seed>\n", argv[0]);
        return 2;
    }
    const std::string kind = argv[1];
    if (kind == "image-check" || kind == "gguf-check") {   // one file as it is, accepted or refused
        uint64_t sink = 0;
        const bool acc = kind == "gguf-check" ? run_gguf(argv[2], sink) : run_image(argv[2], sink);
        printf("ok %d refused %d (sink %016llx)\n", acc ? 1 : 0, acc ? 0 : 1, (unsigned long long) sink);
        return 0;
    }
    const char * scratch = argv[3];
    const long iters = atol(argv[4]);
    rng r(strtoull(argv[5], nullptr, 10));
    std::vector<uint8_t> seed;
    if (!read_all(argv[2], seed) || seed.empty()) { fprintf(stderr, "cannot read %s\n", argv[2]); return 2; }
    size_t hot = 2048, limit = seed.size();
    if (kind == "gguf") {
        gguf::file f;
        std::string err;
        if (!gguf::open(argv[2], f, err)) { fprintf(stderr, "seed does not parse: %s\n", err.c_str()); return 2; }
        limit = (size_t) f.data_offset;   // tensor data is not parsed here
        hot = std::min<size_t>(limit, 256);
    } else if (kind != "image") {
        return 2;
    }
    uint64_t sink = 0;
    long ok = 0, refused = 0;
    if (!write_all(scratch, seed)) return 2;
    const bool seed_ok = kind == "gguf" ? run_gguf(scratch, sink) : run_image(scratch, sink);
    if (!seed_ok) { fprintf(stderr, "the unmutated seed is refused\n"); return 2; }
    for (long i = 0; i < iters; i++) {
        std::vector<uint8_t> d = seed;
        mutate(d, r, hot, limit);
        if (!write_all(scratch, d)) return 2;
        const bool acc = kind == "gguf" ? run_gguf(scratch, sink) : run_image(scratch, sink);
        (acc ? ok : refused)++;
    }
    printf("ok %ld refused %ld (sink %016llx)\n", ok, refused, (unsigned long long) sink);
    return 0;
}
