"""Host-side tooling of the MI355X jepa encoder library: GGUF files, synthetic models, inputs and
the ctypes binding of libjepa.so (the reference's python/src/jepa_cpp/_lib.py role)."""
