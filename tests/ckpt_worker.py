"""GPU half of tests/test_checkpoint.py, run in a child process that never
imports torch: the library's own HIP runtime is then the process's only one,
as in the Rust host.  Writes a Q4/Q6 checkpoint, loads it to device memory
with mh_load_quant (staged reads), copies it back, runs mh_gemv_quant over
the loaded weights and compares both with the source and the oracle.  Prints
one line "OK ..." or raises."""
import ctypes
import pathlib
import sys
import tempfile
import time

sys.modules["torch"] = None  # no torch in this process: its HIP runtime stays out

import numpy as np  # noqa: E402

ROOT = pathlib.Path(__file__).resolve().parent.parent
sys.path.insert(0, str(ROOT))

from molten_amd import hip, layout  # noqa: E402
from oracle import oracle as orc  # noqa: E402
from tests.test_checkpoint import _write_quant  # noqa: E402


def dmalloc(lib, nbytes):
    p = ctypes.c_void_p()
    hip.check(lib.mh_malloc(ctypes.byref(p), nbytes), "malloc")
    return p.value


def h2d(lib, dst, a):
    a = np.ascontiguousarray(a)
    hip.check(lib.mh_memcpy(dst, a.ctypes.data, a.nbytes, 1, None), "memcpy h2d")


def d2h(lib, src, shape, dtype):
    out = np.empty(shape, dtype)
    hip.check(lib.mh_memcpy(out.ctypes.data, src, out.nbytes, 2, None), "memcpy d2h")
    return out


def main(bits: int) -> None:
    lib = hip.load()
    assert all("torch" not in p for p in hip.hip_runtimes()), hip.hip_runtimes()
    rng = np.random.default_rng(bits)
    n, k = 24576, 2048  # Q6 codes 37.7 MB: three 16 MB staging chunks
    h = layout.synth_quant(rng, n, k, bits)
    with tempfile.TemporaryDirectory() as d:
        _write_quant(pathlib.Path(d) / "model.safetensors", "lm_head", h)
        codes = dmalloc(lib, h.codes.nbytes)
        scales = dmalloc(lib, h.scales.nbytes)
        biases = dmalloc(lib, h.biases.nbytes)
        with hip.Checkpoint(d) as ck:
            t0 = time.perf_counter()
            w = ck.load_quant("lm_head", n, k, bits, codes, scales, biases)
            first = time.perf_counter() - t0
            t0 = time.perf_counter()  # again: the staging buffers exist now
            w = ck.load_quant("lm_head", n, k, bits, codes, scales, biases)
            secs = time.perf_counter() - t0
    assert (d2h(lib, codes, h.codes.shape, np.uint32) == h.codes).all(), "codes"
    assert (d2h(lib, scales, h.scales.shape, np.uint16) == h.scales).all(), "scales"
    assert (d2h(lib, biases, h.biases.shape, np.uint16) == h.biases).all(), "biases"
    x = layout.synth_bf16(rng, (1, k))
    dx = dmalloc(lib, x.nbytes)
    dy = dmalloc(lib, n * 2)
    h2d(lib, dx, x)
    hip.gemv_quant(w, dx, dy, 1)
    y = d2h(lib, dy, (1, n), np.uint16)
    assert (y == orc.gemv_quant(h, x, 1)).all(), "gemv over the loaded weights"
    for p in (codes, scales, biases, dx, dy):
        lib.mh_free(p)
    total = h.codes.nbytes + h.scales.nbytes + h.biases.nbytes
    print(f"OK bits={bits} n={n} k={k} loaded {total} B in {secs * 1e3:.1f} ms "
          f"({total / secs / 1e9:.2f} GB/s, file in the page cache; first load {first * 1e3:.1f} ms "
          f"with the staging allocation)", flush=True)


if __name__ == "__main__":
    main(int(sys.argv[1]))
