"""jepa_amd_preprocess_frames_device_noalloc (no counterpart in the reference: preprocessing for callers
that cannot allocate device memory) against jepa_amd_preprocess_frames_device, bit for bit, on two
calls in a row with the second input smaller than the first (the static scratch keeps the first
call's contents), on a caller's stream (a torch stream of its own, not the null stream) and on the
null stream; the call captured into a HIP graph and replayed on new frames; and the refusal of an
input whose scratch would exceed the static array, before any device work."""
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


@pytest.mark.parametrize("use_own_stream", [True, False])
def test_noalloc_equals_allocating_entry_point(jlib, use_own_stream):
    rng = np.random.default_rng(7)
    side = torch.cuda.Stream() if use_own_stream else None
    stream = side.cuda_stream if use_own_stream else None
    if use_own_stream:
        assert stream, "a torch side stream must not be the null stream"
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


def test_noalloc_graph_capture_and_replay(jlib):
    """The call captured on a side stream into a HIP graph (its tables travel as kernel arguments, so
    the graph holds them; there is no host copy and no stream synchronisation to break the capture),
    then replayed three times on new frames written into the same input buffer between replays, each
    replay bit for bit against the allocating entry point on those frames."""
    rng = np.random.default_rng(11)
    T, h, w = 3, 480, 640
    p = _params(jlib, resample=1)
    n_out = 3 * T * 256 * 256
    frames = torch.from_numpy(rng.integers(0, 256, (T, h, w, 3), dtype=np.uint8)).cuda()
    out = torch.full((n_out,), float("nan"), dtype=torch.float32, device="cuda")
    side = torch.cuda.Stream()
    oh, ow = C.c_int(0), C.c_int(0)
    fn = jlib.lib().jepa_amd_preprocess_frames_device_noalloc
    args = lambda st: [0, C.byref(p), frames.data_ptr(), T, h, w, out.data_ptr(), out.numel(), C.byref(oh), C.byref(ow), st]
    torch.cuda.synchronize()
    # one eager call first: the per-device scratch address is looked up outside the capture
    with torch.cuda.stream(side):
        assert fn(*args(side.cuda_stream)) == 0, jlib.error_text()
    side.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=side):
        rc = fn(*args(side.cuda_stream))
    assert rc == 0, jlib.error_text()
    for rep in range(3):
        new = rng.integers(0, 256, (T, h, w, 3), dtype=np.uint8)
        frames.copy_(torch.from_numpy(new).cuda())
        out.fill_(float("nan"))
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        got = out.cpu().numpy()
        want, _ = _run(jlib, "jepa_amd_preprocess_frames_device", p, frames, T, h, w, n_out)
        assert np.isfinite(want).all()
        np.testing.assert_array_equal(got.view(np.uint32), want.view(np.uint32), err_msg=f"replay {rep}")
    del g


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
