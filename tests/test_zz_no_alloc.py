"""jepa_amd_preprocess_frames_device_noalloc (no counterpart in the reference: preprocessing for callers
that cannot allocate device memory) against jepa_amd_preprocess_frames_device, bit for bit, on two
calls in a row with the second input smaller than the first (the static scratch keeps the first
call's contents), on the caller's stream and on the null stream; and the refusal of an input whose
scratch would exceed the static array, before any device work."""
import ctypes as C

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")


def _params(jlib, resize_short=256, crop=256, resample=0):
    p = jlib.PreprocessParams()
    for c, (m, sd) in enumerate(zip((0.485, 0.456, 0.406), (0.229, 0.224, 0.225))):
        p.mean[c], p.std[c] = m, sd
    p.resize_short, p.crop, p.resample, p.resize_mode, p.rescale, p.fused_norm = resize_short, crop, resample, 0, 1.0 / 255.0, True
    return p


def _run(jlib, fn, p, frames_dev, T, h, w, n_out, stream=None):
    out = torch.full((n_out,), float("nan"), dtype=torch.float32, device="cuda")
    torch.cuda.synchronize()
    oh, ow = C.c_int(0), C.c_int(0)
    args = [0, C.byref(p), frames_dev.data_ptr(), T, h, w, out.data_ptr(), out.numel(), C.byref(oh), C.byref(ow)]
    if fn == "jepa_amd_preprocess_frames_device_noalloc":
        args.append(stream)
    rc = getattr(jlib.lib(), fn)(*args)
    assert rc == 0, jlib.error_text()
    torch.cuda.synchronize()
    return out.cpu().numpy(), (oh.value, ow.value)


@pytest.mark.parametrize("use_torch_stream", [True, False])
def test_noalloc_equals_allocating_entry_point(jlib, use_torch_stream):
    rng = np.random.default_rng(7)
    stream = torch.cuda.current_stream().cuda_stream if use_torch_stream else None
    # first a larger input, then a smaller one: the second call must not see the first one's scratch
    for (T, h, w, resample) in [(4, 720, 1280, 1), (2, 300, 400, 0)]:
        frames = torch.from_numpy(rng.integers(0, 256, (T, h, w, 3), dtype=np.uint8)).cuda()
        p = _params(jlib, resample=resample)
        n_out = 3 * T * 256 * 256
        want, shape_a = _run(jlib, "jepa_amd_preprocess_frames_device", p, frames, T, h, w, n_out)
        got, shape_b = _run(jlib, "jepa_amd_preprocess_frames_device_noalloc", p, frames, T, h, w, n_out, stream)
        assert shape_a == shape_b == (256, 256)
        assert np.isfinite(want).all()
        np.testing.assert_array_equal(got.view(np.uint32), want.view(np.uint32))


def test_noalloc_refuses_oversized_scratch(jlib):
    # 64 frames of 1080 x 1920 cropped to 256: the horizontal pass alone is 64 * 1080 * 256 * 3 bytes,
    # over the 32 MiB static array; refused on the host, before any device work
    # (the buffers have the sizes the call describes, so nothing could go out of bounds either way)
    p = _params(jlib)
    frames = torch.zeros((64, 1080, 1920, 3), dtype=torch.uint8, device="cuda")
    out = torch.zeros(3 * 64 * 256 * 256, dtype=torch.float32, device="cuda")
    torch.cuda.synchronize()
    jlib.lib().jepa_error_reset()
    rc = jlib.lib().jepa_amd_preprocess_frames_device_noalloc(0, C.byref(p), frames.data_ptr(), 64, 1080, 1920, out.data_ptr(),
                                                             out.numel(), None, None, None)
    assert rc == -1
    assert "scratch" in jlib.error_text()
