"""The boundary contracts of include/jepa.h that need a GPU:

- threading (include/jepa.h:612-647, reference tests/test-threads.cpp:1-25): one model shared by
  several threads, each with its own context, gives exactly the results of serial calls;
- the activation budget (reference tests/test-ops.cpp:401-435): with $JEPA_MAX_GRAPH_MIB = 1 at
  context creation a 16-frame clip is refused with a message naming the knob, and without it the
  same model encodes.
"""
import threading

import numpy as np
import pytest

from jepa_amd import forge, inputs

pytestmark = pytest.mark.gpu


def test_contexts_in_threads_equal_serial(jlib, models_dir):
    cfg = forge.tiny("vjepa2", "q8_0", embed_dim=256, n_head=4, ffn_dim=1024)
    m = jlib.Model(forge.cached_model(cfg, models_dir))
    xs = [inputs.make_input(1, 8, 128, 128, seed=100 + i) for i in range(4)]
    serial = [jlib.Context(m).encode(x) for x in xs]
    results, errors = {}, []

    def work(i):
        try:
            ctx = jlib.Context(m)
            results[i] = [ctx.encode(xs[i]) for _ in range(4)]
        except Exception as e:          # reported below, in the main thread
            errors.append(repr(e))

    threads = [threading.Thread(target=work, args=(i,)) for i in range(len(xs))]
    for t in threads:
        t.start()
    for t in threads:
        t.join()
    assert not errors, errors
    for i, outs in results.items():
        for o in outs:
            np.testing.assert_array_equal(o.view(np.uint32), serial[i].view(np.uint32))
    # and the inputs really differ, so a mix-up between threads would show
    assert not np.array_equal(serial[0], serial[1])


def test_graph_budget_refusal(jlib, models_dir, monkeypatch):
    m = jlib.Model(forge.cached_model(forge.tiny("vjepa2", "q8_0"), models_dir))
    monkeypatch.setenv("JEPA_MAX_GRAPH_MIB", "1")
    ctx = jlib.Context(m)                  # the context reads the budget when it is created
    with pytest.raises(RuntimeError) as e:
        ctx.encode(inputs.make_input(1, 16, 256, 256, seed=1))
    assert "JEPA_MAX_GRAPH_MIB" in str(e.value)
    monkeypatch.delenv("JEPA_MAX_GRAPH_MIB")
    ctx2 = jlib.Context(m)
    out = ctx2.encode(inputs.make_input(1, 2, 64, 64, seed=1))
    assert out.shape[0] == m.token_grid(2, 64, 64) > 0
    assert np.isfinite(out).all()
