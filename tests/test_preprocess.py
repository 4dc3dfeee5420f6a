"""Host preprocessing behind include/jepa.h (reference src/preprocess.cpp), no GPU:

- jepa_resize_antialias_u8 against PyTorch's own CPU kernel for the uint8 antialiased resize
  (torch.nn.functional.interpolate on uint8 with antialias=True, channels-last: the kernel the
  reference ports, src/preprocess.cpp:1-10), bit for bit, bilinear and bicubic, down and up;
- the crop / normalisation pipeline (jepa_preprocess_frames_rgb_ex) against a numpy restatement
  on top of that resize, bit for bit;
- jepa_load_image_rgb against PIL: PNG (every colour type and bit depth, Adam7, all five row
  filters through a test-side encoder), PPM / PGM, and baseline JPEG (4:4:4, 4:2:2, 4:2:0, grey,
  and the reference's own COCO fixture) with libjpeg's default decoding; progressive JPEG refused.
"""
import ctypes as C
import io
import os
import struct
import zlib

import numpy as np
import pytest
import torch
import torch.nn.functional as F
from PIL import Image

from jepa_amd import _lib

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "media")


def torch_resize(img, oh, ow, mode):
    x = torch.from_numpy(np.array(img, copy=True)).permute(2, 0, 1)[None].contiguous(memory_format=torch.channels_last)
    y = F.interpolate(x, size=(oh, ow), mode=mode, antialias=True)
    return y[0].permute(1, 2, 0).contiguous().numpy()


RESIZE_CASES = [((37, 53), (17, 29)), ((480, 640), (224, 298)), ((224, 300), (224, 298)), ((300, 224), (298, 224)),
                ((100, 80), (300, 240)), ((5, 1), (7, 3)), ((1080, 1920), (224, 398)), ((256, 256), (224, 224))]


@pytest.mark.parametrize("resample,mode", [(0, "bilinear"), (1, "bicubic")])
@pytest.mark.parametrize("src,dst", RESIZE_CASES)
def test_resize_matches_torch_uint8_antialias(src, dst, resample, mode):
    rng = np.random.default_rng(src[0] * 7 + dst[1] + resample)
    # smooth content plus noise, so both the filter shape and the rounding are exercised
    yy, xx = np.mgrid[0:src[0], 0:src[1]]
    base = (127 + 100 * np.sin(yy / 7.0)[..., None] * np.cos(xx / 11.0)[..., None]) + rng.normal(0, 20, (src[0], src[1], 3))
    img = np.clip(base, 0, 255).astype(np.uint8)
    got = _lib.resize_u8(img, dst[0], dst[1], resample)
    want = torch_resize(img, dst[0], dst[1], mode)
    assert np.array_equal(got, want), f"{int((got != want).sum())} of {got.size} bytes differ"


def test_resize_identity_copies():
    img = np.random.default_rng(0).integers(0, 256, (31, 17, 3), dtype=np.uint8)
    assert np.array_equal(_lib.resize_u8(img, 31, 17, 1), img)


def _params(resize_short=224, crop=224, resample=0, mode=0, fused=True, rescale=1.0 / 255.0):
    p = _lib.PreprocessParams()
    for c, (m, s) in enumerate(zip((0.485, 0.456, 0.406), (0.229, 0.224, 0.225))):
        p.mean[c], p.std[c] = m, s
    p.resize_short, p.crop, p.resample, p.resize_mode, p.rescale, p.fused_norm = resize_short, crop, resample, mode, rescale, fused
    return p


def _pipeline_ref(p, frames):
    """numpy restatement of reference src/preprocess.cpp:202-300 on top of the torch resize"""
    h, w, _ = frames[0].shape
    if p.resize_mode == 1:
        rh = rw = p.resize_short
    elif w <= h:
        rw, rh = p.resize_short, p.resize_short * h // w
    else:
        rh, rw = p.resize_short, p.resize_short * w // h
    crop = p.crop if p.crop > 0 else min(rh, rw)
    inv = 1.0 / float(np.float32(p.rescale))
    if abs(inv - round(inv)) < 1e-3 * abs(inv):
        inv = float(round(inv))
    inv = np.float32(inv)
    out = np.zeros((3, len(frames), crop, crop), np.float32)
    for t, f in enumerate(frames):
        r = torch_resize(f, rh, rw, "bicubic" if p.resample == 1 else "bilinear")
        nh, nw = max(crop, rh), max(crop, rw)
        pt, pl = (crop - rh) // 2 if crop > rh else 0, (crop - rw) // 2 if crop > rw else 0
        pad = np.zeros((nh, nw, 3), np.uint8)
        pad[pt:pt + rh, pl:pl + rw] = r
        top, left = (nh - crop) // 2, (nw - crop) // 2
        c8 = pad[top:top + crop, left:left + crop].astype(np.float32)
        for c in range(3):
            mean, std = np.float32(p.mean[c]), np.float32(p.std[c])
            if p.fused_norm:
                out[c, t] = (c8[..., c] - mean * inv) / (std * inv)
            else:
                out[c, t] = (c8[..., c] / inv - mean) / std
    return out


PIPE_CASES = [dict(), dict(resample=1), dict(mode=1, resize_short=200, crop=200), dict(crop=0), dict(crop=320),
              dict(fused=False), dict(resize_short=96, crop=128, resample=1)]


@pytest.mark.parametrize("kw", PIPE_CASES)
@pytest.mark.parametrize("hw", [(360, 480), (480, 360), (224, 224)])
def test_preprocess_frames_matches_restatement(kw, hw):
    rng = np.random.default_rng(hw[0] + len(kw))
    frames = [rng.integers(0, 256, (hw[0], hw[1], 3), dtype=np.uint8) for _ in range(2)]
    p = _params(**kw)
    got = _lib.preprocess_frames(p, frames)
    want = _pipeline_ref(p, frames)
    assert got.shape == want.shape
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))


def test_preprocess_rejects_bad_params():
    f = np.zeros((10, 10, 3), np.uint8)
    for bad in (_params(resize_short=0), _params(rescale=0.0)):
        with pytest.raises(RuntimeError):
            _lib.preprocess_frames(bad, [f])
    p = _params()
    p.std[1] = 0.0
    with pytest.raises(RuntimeError):
        _lib.preprocess_frames(p, [f])
    # an aspect ratio whose shortest-edge intermediate is over the 64-megapixel cap
    with pytest.raises(RuntimeError):
        _lib.preprocess_frames(_params(resize_short=224), [np.zeros((1, 400000, 3), np.uint8)])


# ------------------------------------------------------------------------------------------------ PNG
def _png(path, arr, ctype, depth, interlace=False, palette=None, seed=0):
    """PNG writer with a random row filter per row (all five filter types) and optional Adam7"""
    rng = np.random.default_rng(seed)
    chans = {0: 1, 2: 3, 3: 1, 4: 2, 6: 4}[ctype]
    H, W = arr.shape[:2]
    def rows_of(sub):
        h, w = sub.shape[:2]
        if depth == 16:
            data = sub.astype(">u2").reshape(h, w * chans).view(np.uint8).reshape(h, -1)
        elif depth == 8:
            data = sub.reshape(h, w * chans).astype(np.uint8)
        else:
            bits = np.unpackbits(sub.reshape(h, w, 1).astype(np.uint8), axis=2)[:, :, 8 - depth:].reshape(h, w * depth)
            pad = (-bits.shape[1]) % 8
            data = np.packbits(np.pad(bits, ((0, 0), (0, pad))), axis=1)
        bpp = max(1, chans * depth // 8)
        out = bytearray()
        prev = np.zeros(data.shape[1], np.int32)
        for y in range(h):
            cur = data[y].astype(np.int32)
            ft = int(rng.integers(0, 5))
            a = np.concatenate([np.zeros(bpp, np.int32), cur[:-bpp]])
            c = np.concatenate([np.zeros(bpp, np.int32), prev[:-bpp]])
            if ft == 0: f = cur
            elif ft == 1: f = cur - a
            elif ft == 2: f = cur - prev
            elif ft == 3: f = cur - (a + prev) // 2
            else:
                p = a + prev - c
                pa, pb, pc = np.abs(p - a), np.abs(p - prev), np.abs(p - c)
                f = cur - np.where((pa <= pb) & (pa <= pc), a, np.where(pb <= pc, prev, c))
            out += bytes([ft]) + (f & 255).astype(np.uint8).tobytes()
            prev = cur
        return bytes(out)
    if interlace:
        raw = b""
        for x0, y0, dx, dy in ((0, 0, 8, 8), (4, 0, 8, 8), (0, 4, 4, 8), (2, 0, 4, 4), (0, 2, 2, 4), (1, 0, 2, 2), (0, 1, 1, 2)):
            sub = arr[y0::dy, x0::dx]
            if sub.shape[0] and sub.shape[1]:
                raw += rows_of(sub)
    else:
        raw = rows_of(arr)
    def chunk(t, d):
        return struct.pack(">I", len(d)) + t + d + struct.pack(">I", zlib.crc32(t + d) & 0xffffffff)
    png = b"\x89PNG\r\n\x1a\n" + chunk(b"IHDR", struct.pack(">IIBBBBB", W, H, depth, ctype, 0, 0, 1 if interlace else 0))
    if palette is not None:
        png += chunk(b"PLTE", palette.astype(np.uint8).tobytes())
    png += chunk(b"IDAT", zlib.compress(raw)) + chunk(b"IEND", b"")
    open(path, "wb").write(png)


@pytest.mark.parametrize("interlace", [False, True])
@pytest.mark.parametrize("kind", ["rgb8", "rgba8", "grey8", "greya8", "rgb16", "grey16", "pal8", "pal4", "grey1", "grey2"])
def test_png_decoder(tmp_path, kind, interlace):
    rng = np.random.default_rng(len(kind) + interlace)
    H, W = 23, 37
    pal = None
    if kind == "rgb8": arr, ct, d = rng.integers(0, 256, (H, W, 3)), 2, 8
    elif kind == "rgba8": arr, ct, d = rng.integers(0, 256, (H, W, 4)), 6, 8
    elif kind == "grey8": arr, ct, d = rng.integers(0, 256, (H, W, 1)), 0, 8
    elif kind == "greya8": arr, ct, d = rng.integers(0, 256, (H, W, 2)), 4, 8
    elif kind == "rgb16": arr, ct, d = rng.integers(0, 65536, (H, W, 3)), 2, 16
    elif kind == "grey16": arr, ct, d = rng.integers(0, 65536, (H, W, 1)), 0, 16
    elif kind == "pal8": arr, ct, d, pal = rng.integers(0, 200, (H, W, 1)), 3, 8, rng.integers(0, 256, (200, 3))
    elif kind == "pal4": arr, ct, d, pal = rng.integers(0, 16, (H, W, 1)), 3, 4, rng.integers(0, 256, (16, 3))
    elif kind == "grey1": arr, ct, d = rng.integers(0, 2, (H, W, 1)), 0, 1
    else: arr, ct, d = rng.integers(0, 4, (H, W, 1)), 0, 2
    path = str(tmp_path / f"{kind}.png")
    _png(path, arr, ct, d, interlace, pal, seed=W)
    got = _lib.load_image(path)
    if ct == 3:
        want = pal[arr[..., 0]]
    elif d == 16:
        want = arr >> 8
    elif d < 8:
        want = arr * (255 // ((1 << d) - 1))
    else:
        want = arr
    want = want[..., :3] if want.shape[2] >= 3 else np.repeat(want[..., :1], 3, axis=2)
    assert np.array_equal(got, want.astype(np.uint8))
    if not interlace and kind in ("rgb8", "rgba8", "grey8", "pal8"):   # and PIL agrees
        assert np.array_equal(got, np.asarray(Image.open(path).convert("RGB")))


def test_pnm_decoder(tmp_path):
    rng = np.random.default_rng(5)
    rgb = rng.integers(0, 256, (13, 21, 3), dtype=np.uint8)
    grey = rng.integers(0, 256, (13, 21), dtype=np.uint8)
    (tmp_path / "a.ppm").write_bytes(b"P6\n# comment\n21 13\n255\n" + rgb.tobytes())
    (tmp_path / "b.pgm").write_bytes(b"P5 21 13 255\n" + grey.tobytes())
    assert np.array_equal(_lib.load_image(str(tmp_path / "a.ppm")), rgb)
    assert np.array_equal(_lib.load_image(str(tmp_path / "b.pgm")), np.repeat(grey[..., None], 3, axis=2))


# ------------------------------------------------------------------------------------------------ JPEG
def _photo(h, w, seed):
    rng = np.random.default_rng(seed)
    yy, xx = np.mgrid[0:h, 0:w]
    img = np.stack([128 + 90 * np.sin(yy / 9.0 + c) * np.cos(xx / 13.0 - c) for c in range(3)], -1) + rng.normal(0, 12, (h, w, 3))
    return np.clip(img, 0, 255).astype(np.uint8)


@pytest.mark.parametrize("subsampling", [0, 1, 2])
@pytest.mark.parametrize("hw", [(64, 96), (67, 101), (8, 8), (121, 17)])
def test_jpeg_decoder_matches_libjpeg_default(tmp_path, subsampling, hw):
    """Baseline JPEG written by PIL (libjpeg), decoded here and by PIL with its defaults (islow IDCT,
    fancy upsampling): the same pixels."""
    path = str(tmp_path / "x.jpg")
    Image.fromarray(_photo(*hw, seed=hw[1])).save(path, quality=90, subsampling=subsampling)
    got = _lib.load_image(path)
    want = np.asarray(Image.open(path).convert("RGB"))
    assert got.shape == want.shape
    diff = np.abs(got.astype(int) - want.astype(int))
    assert diff.max() == 0, f"max diff {diff.max()}, {int((diff > 0).sum())} values"


def test_jpeg_decoder_grey_and_restarts(tmp_path):
    path = str(tmp_path / "g.jpg")
    Image.fromarray(_photo(50, 70, 3)[..., 0]).save(path, quality=85)
    assert np.array_equal(_lib.load_image(path), np.asarray(Image.open(path).convert("RGB")))
    # restart markers every 2 MCU rows (DRI + RSTn handling)
    path = str(tmp_path / "r.jpg")
    try:
        Image.fromarray(_photo(80, 96, 4)).save(path, quality=90, subsampling=2, restart_marker_rows=2)
    except TypeError:
        pytest.skip("this PIL cannot write restart markers")
    assert b"\xff\xdd" in open(path, "rb").read()
    assert np.array_equal(_lib.load_image(path), np.asarray(Image.open(path).convert("RGB")))


def test_jpeg_progressive_is_refused(tmp_path):
    path = str(tmp_path / "p.jpg")
    Image.fromarray(_photo(32, 32, 1)).save(path, quality=90, progressive=True)
    with pytest.raises(RuntimeError, match="progressive"):
        _lib.load_image(path)


COCO = sorted(f for f in os.listdir(GOLDEN) if f.startswith("coco_") and f.endswith(".jpg"))


@pytest.mark.parametrize("name", COCO)
def test_reference_fixture_jpeg(name):
    """The eight COCO photos of the reference's tests/fixtures/media (what its test-batch and parity
    tests encode): decoded pixels equal PIL's (libjpeg) bit for bit, and so does the whole file
    pipeline (jepa_preprocess_image_file with the library defaults)."""
    path = os.path.join(GOLDEN, name)
    got = _lib.load_image(path)
    want = np.asarray(Image.open(path).convert("RGB"))
    assert np.array_equal(got, want)
    # and the whole file pipeline (jepa_preprocess_image_file with the library defaults)
    L = _lib.lib()
    oh, ow = C.c_int(0), C.c_int(0)
    r = L.jepa_preprocess_image_file(None, path.encode(), C.byref(oh), C.byref(ow))
    assert r
    out = np.ctypeslib.as_array(r, shape=(3 * oh.value * ow.value,)).copy().reshape(3, 1, oh.value, ow.value)
    L.jepa_free(C.cast(r, C.c_void_p))
    p = L.jepa_preprocess_default_params(None)
    assert np.array_equal(out.view(np.uint32), _pipeline_ref(p, [want]).view(np.uint32))


def test_load_image_errors(tmp_path):
    (tmp_path / "junk.bin").write_bytes(b"not an image at all")
    for path in (str(tmp_path / "missing.png"), str(tmp_path / "junk.bin")):
        with pytest.raises(RuntimeError):
            _lib.load_image(path)
    buf = io.BytesIO()
    Image.fromarray(_photo(16, 16, 2)).save(buf, format="PNG")
    (tmp_path / "cut.png").write_bytes(buf.getvalue()[:60])
    with pytest.raises(RuntimeError):
        _lib.load_image(str(tmp_path / "cut.png"))
