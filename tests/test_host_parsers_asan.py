"""The host-side parsers of untrusted files under AddressSanitizer and UndefinedBehaviorSanitizer (CPU,
no GPU): tests/host_parsers_fuzz.cpp, built with g++ from the library's own image_io.cpp,
jpeg_decode.cpp, gguf.cpp and preprocess.cpp, runs a seeded mutation campaign (bit flips, boundary
values in 32- and 64-bit fields of either byte order, truncations, copied chunks) over:

- the golden JPEG (tests/golden/media), through jepa_load_image_rgb and, for what decodes, the
  preprocessing and the antialiased resize;
- PNGs of every colour type the decoder reads (grey 1 and 8 bit, palette 4 bit, grey + alpha,
  RGB 8 bit plain and Adam7-interlaced, RGBA 16 bit) and binary PGM / PPM, written here;
- a small GGUF model file written by the forge, its header, metadata and tensor table, through
  gguf::open.

Any sanitizer report aborts the program and fails the test. The campaign caught two signed
overflows in the PNG / PNM size checks (two 32-bit header sizes multiplied in int64), which let a
hostile header slip past the pixel limit; both are fixed and stay covered here."""
import os
import shutil
import struct
import subprocess
import zlib

import numpy as np
import pytest

from jepa_amd import forge

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
CSRC = os.path.join(ROOT, "jepa.cpp_amd", "csrc")
HIP_INCLUDE = "/opt/rocm/include"
JPEG = os.path.join(ROOT, "tests", "golden", "media", "coco_000000000724.jpg")

pytestmark = pytest.mark.skipif(shutil.which("g++") is None or not os.path.isdir(os.path.join(HIP_INCLUDE, "hip")),
                                reason="needs g++ and the HIP headers")

# Adam7 passes: x0, y0, dx, dy
ADAM7 = [(0, 0, 8, 8), (4, 0, 8, 8), (0, 4, 4, 8), (2, 0, 4, 4), (0, 2, 2, 4), (1, 0, 2, 2), (0, 1, 1, 2)]


def _png(rng, w, h, ctype, depth, interlace):
    """A PNG of random pixels with every row filter type (0-4 by row)."""
    bits = {0: 1, 2: 3, 3: 1, 4: 2, 6: 4}[ctype] * depth

    def rows(pw, ph):
        rb = (pw * bits + 7) // 8
        return b"".join(bytes([y % 5]) + rng.integers(0, 256, rb, dtype=np.uint8).tobytes() for y in range(ph))

    if interlace:
        raw = b"".join(rows((w - x0 + dx - 1) // dx, (h - y0 + dy - 1) // dy) for x0, y0, dx, dy in ADAM7
                       if w > x0 and h > y0)
    else:
        raw = rows(w, h)

    def chunk(t, d):
        return struct.pack(">I", len(d)) + t + d + struct.pack(">I", zlib.crc32(t + d) & 0xFFFFFFFF)

    s = b"\x89PNG\r\n\x1a\n" + chunk(b"IHDR", struct.pack(">IIBBBBB", w, h, depth, ctype, 0, 0, interlace))
    if ctype == 3:
        s += chunk(b"PLTE", rng.integers(0, 256, 3 * 16, dtype=np.uint8).tobytes())
    return s + chunk(b"IDAT", zlib.compress(raw)) + chunk(b"IEND", b"")


@pytest.fixture(scope="module")
def fuzzer(tmp_path_factory):
    d = tmp_path_factory.mktemp("asan")
    exe = d / "host_parsers_fuzz"
    srcs = [os.path.join(ROOT, "tests", "host_parsers_fuzz.cpp")] + \
           [os.path.join(CSRC, f) for f in ("image_io.cpp", "jpeg_decode.cpp", "gguf.cpp", "preprocess.cpp")]
    cmd = ["g++", "-std=c++17", "-O1", "-g", "-fsanitize=address,undefined", "-fno-sanitize-recover=all",
           "-fno-omit-frame-pointer", "-D__HIP_PLATFORM_AMD__", "-I", HIP_INCLUDE, "-I", os.path.join(ROOT, "include"),
           "-I", CSRC, *srcs, "-lz", "-o", str(exe)]
    r = subprocess.run(cmd, capture_output=True, text=True)
    assert r.returncode == 0, r.stderr[-3000:]
    return str(exe), d


def _campaign(fuzzer, kind, seed_path, iters, seed):
    exe, d = fuzzer
    print(f"campaign: {kind} {os.path.basename(str(seed_path))} x {iters}, rng seed {seed}", flush=True)
    env = dict(os.environ, ASAN_OPTIONS="detect_leaks=1:abort_on_error=0", UBSAN_OPTIONS="print_stacktrace=1")
    r = subprocess.run([exe, kind, str(seed_path), str(d / f"scratch_{seed}.bin"), str(iters), str(seed)],
                       capture_output=True, text=True, timeout=600, env=env)
    assert r.returncode == 0, (os.path.basename(str(seed_path)), r.stdout[-1000:], r.stderr[-4000:])
    ok, refused = (int(v) for v in r.stdout.split()[1:4:2])
    print(f"{kind} {os.path.basename(str(seed_path))}: {ok} accepted, {refused} refused of {iters} mutations")
    assert ok + refused == iters
    return ok, refused


def test_jpeg(fuzzer):
    ok, refused = _campaign(fuzzer, "image", JPEG, 300, 7919)
    assert ok > 0 and refused > 0


@pytest.mark.parametrize("name,shape", [("grey1", (29, 7, 0, 1, 0)), ("grey8", (19, 31, 0, 8, 0)), ("pal4", (33, 9, 3, 4, 0)),
                                        ("ga8", (11, 13, 4, 8, 0)), ("rgb8", (37, 23, 2, 8, 0)),
                                        ("rgb8_adam7", (21, 19, 2, 8, 1)), ("rgba16", (9, 17, 6, 16, 0))])
def test_png(fuzzer, name, shape):
    p = fuzzer[1] / f"{name}.png"
    p.write_bytes(_png(np.random.default_rng(len(name)), *shape))
    _campaign(fuzzer, "image", p, 1500, 3)


def test_pnm(fuzzer):
    rng = np.random.default_rng(5)
    p6, p5 = fuzzer[1] / "seed.ppm", fuzzer[1] / "seed.pgm"
    p6.write_bytes(b"P6\n# comment\n23 17\n255\n" + rng.integers(0, 256, 23 * 17 * 3, dtype=np.uint8).tobytes())
    p5.write_bytes(b"P5 13 11 200\n" + rng.integers(0, 201, 13 * 11, dtype=np.uint8).tobytes())
    for p in (p6, p5):
        ok, refused = _campaign(fuzzer, "image", p, 1500, 11)
        assert ok > 0 and refused > 0


def test_gguf(fuzzer):
    cfg = forge.tiny("vjepa2", "q8_0", n_classes=10, n_pool_layers=1, pred_dim=128, pred_layers=1, pred_ffn=512)
    p = fuzzer[1] / "seed.gguf"
    forge.write_model(cfg, str(p))
    ok, refused = _campaign(fuzzer, "gguf", p, 2000, 13)
    assert ok > 0 and refused > 0


def _chunk(t, d):
    return struct.pack(">I", len(d)) + t + d + struct.pack(">I", zlib.crc32(t + d) & 0xFFFFFFFF)


@pytest.mark.parametrize("name,data", [
    # 0xFFFFFFFF x 0xFFFFFFFF: the product of the two sizes overflowed int64 and came out negative,
    # under the pixel limit
    ("png_huge_ihdr", b"\x89PNG\r\n\x1a\n" + _chunk(b"IHDR", struct.pack(">IIBBBBB", 0xFFFFFFFF, 0xFFFFFFFF, 8, 2, 0, 0, 0))
     + _chunk(b"IDAT", zlib.compress(b"\0" * 64)) + _chunk(b"IEND", b"")),
    ("png_huge_ihdr_adam7", b"\x89PNG\r\n\x1a\n" + _chunk(b"IHDR", struct.pack(">IIBBBBB", 0xFFFFFFFF, 0xFFFFFF7F, 16, 6, 0, 0, 1))
     + _chunk(b"IDAT", zlib.compress(b"\0" * 64)) + _chunk(b"IEND", b"")),
    # sizes of eleven digits (the header parser stops a number past 2^30, at up to ~2^33.3)
    ("ppm_huge_sizes", b"P6 10737418239 10737418239 255\n" + b"\0" * 64),
    ("pgm_one_huge_side", b"P5 1 10737418239 255\n" + b"\0" * 64),
], ids=["png_huge_ihdr", "png_huge_ihdr_adam7", "ppm_huge_sizes", "pgm_one_huge_side"])
def test_hostile_headers_refused(fuzzer, name, data):
    """Regression files for the size-product overflows: refused with a message, no sanitizer report."""
    p = fuzzer[1] / name
    p.write_bytes(data)
    exe, _ = fuzzer
    r = subprocess.run([exe, "image-check", str(p), "-", "0", "0"], capture_output=True, text=True, timeout=60)
    assert r.returncode == 0, (name, r.stdout[-1000:], r.stderr[-4000:])
    assert r.stdout.startswith("ok 0 refused 1"), r.stdout
