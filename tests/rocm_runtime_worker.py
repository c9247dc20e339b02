"""Hot-path parity on the HIP runtime a host without torch binds (the Rust
host of the integration guide links /opt/rocm's libamdhip64): run in a child
process in which torch cannot be imported, so the library loads the ROCm
runtime alone.  Device memory comes from mh_malloc, copies from mh_memcpy,
streams are the default one.  Full-size BASELINE configurations against the
oracle:

- config 1: Q4 GEMV 2048 x 2048, the logits bit-exact;
- config 2: Q4 LM head 65536 x 2048 + argmax, logits and id bit-exact;
- config 5: Q6 LM head 65536 x 2048 at batch 1 (logits and id bit-exact)
  and batch 8 (ids exact, logits within rel-L2 <= 5e-3 and max abs err
  <= 2e-2 x max |ref|: the matrix-core kernel);
- config 3: the MoE decode step (router bf16 2048 x 64, softmax top-4,
  64 Q4 experts 1536 x 2048 / 2048 x 1536), every output bit-exact, over
  three steps sharing one scratch.

Prints one "OK ..." line per configuration and "OK runtime <path>", or
raises."""
import ctypes
import pathlib
import sys

sys.modules["torch"] = None  # no torch in this process: its HIP runtime stays out

import numpy as np  # noqa: E402

ROOT = pathlib.Path(__file__).resolve().parent.parent
sys.path.insert(0, str(ROOT))

from molten_amd import hip, layout  # noqa: E402
from oracle import oracle as orc  # noqa: E402


class Dev:
    """A device buffer from mh_malloc (data_ptr / element_size like a tensor)."""

    def __init__(self, lib, nbytes: int, itemsize: int = 1):
        self.lib, self.itemsize = lib, itemsize
        p = ctypes.c_void_p()
        hip.check(lib.mh_malloc(ctypes.byref(p), max(nbytes, 1)), "malloc")
        self.p, self.nbytes = p.value, nbytes

    def data_ptr(self) -> int:
        return self.p

    def element_size(self) -> int:
        return self.itemsize

    def free(self) -> None:
        self.lib.mh_free(self.p)


def up(lib, a: np.ndarray) -> Dev:
    a = np.ascontiguousarray(a)
    d = Dev(lib, a.nbytes, a.itemsize)
    hip.check(lib.mh_memcpy(d.p, a.ctypes.data, a.nbytes, 1, None), "memcpy h2d")
    return d


def down(lib, d: Dev, shape, dtype) -> np.ndarray:
    out = np.empty(shape, dtype)
    hip.check(lib.mh_memcpy(out.ctypes.data, d.p, out.nbytes, 2, None), "memcpy d2h")
    return out


def zeros(lib, nbytes: int, itemsize: int = 1) -> Dev:
    d = Dev(lib, nbytes, itemsize)
    hip.check(lib.mh_zero(d.p, nbytes, None), "zero")
    return d


def quant(lib, h):
    bufs = [up(lib, h.codes), up(lib, h.scales), up(lib, h.biases)]
    w = hip.QuantWeights(bufs[0].p, bufs[1].p, bufs[2].p, h.n, h.k, h.group_size, h.bits)
    return w, bufs


def within_tolerance(got: np.ndarray, want: np.ndarray, name: str) -> None:
    g = layout.bf16_to_f32(got).astype(np.float64)
    w = layout.bf16_to_f32(want).astype(np.float64)
    assert np.isfinite(g).all(), f"{name}: non-finite outputs"
    rel = float(np.linalg.norm(g - w) / max(np.linalg.norm(w), 1e-30))
    mx = float(np.abs(g - w).max())
    assert rel <= 5e-3 and mx <= 2e-2 * max(float(np.abs(w).max()), 1.0), (name, rel, mx)
    print(f"   {name}: rel-L2 {rel:.3g}, max abs err {mx:.4g} (max |ref| {np.abs(w).max():.4g})", flush=True)


def heads(lib, rng) -> None:
    for name, n, bits, batch in (("config1", 2048, 4, 1), ("config2", 65536, 4, 1),
                                 ("config5_b1", 65536, 6, 1), ("config5_b8", 65536, 6, 8)):
        h = layout.synth_quant(rng, n, 2048, bits)
        x = layout.synth_bf16(rng, (batch, 2048))
        w, keep = quant(lib, h)
        dx = up(lib, x)
        dy = Dev(lib, batch * n * 2, 2)
        want = orc.gemv_quant(h, x, batch)
        if name == "config1":
            hip.gemv_quant(w, dx, dy, 1)
            hip.check(lib.mh_stream_synchronize(None), "sync")
            assert np.array_equal(down(lib, dy, (1, n), np.uint16), want), name
        else:
            scratch = zeros(lib, hip.argmax_scratch_words(batch) * 8, 8)
            ids = Dev(lib, batch * 4, 4)
            for step in range(2):  # the second call reuses the scratch the first left
                hip.gemv_quant_argmax(w, dx, dy, scratch, ids, batch)
                hip.check(lib.mh_stream_synchronize(None), "sync")
                got = down(lib, dy, (batch, n), np.uint16)
                got_ids = down(lib, ids, (batch,), np.uint32)
                want_ids = [orc.argmax_bf16(want[b]) for b in range(batch)]
                assert got_ids.tolist() == want_ids, (name, step, got_ids.tolist(), want_ids)
                if batch == 1:
                    assert np.array_equal(got, want), (name, step)
                else:
                    within_tolerance(got, want, f"{name} logits")
            scratch.free()
            ids.free()
        for d in keep + [dx, dy]:
            d.free()
        print(f"OK {name} {n}x2048 Q{bits} batch {batch}", flush=True)


def moe_decode(lib, rng) -> None:
    E, H, I, TOPK = 64, 2048, 1536, 4
    gate = layout.synth_quant(rng, E * I, H, 4)
    upw = layout.synth_quant(rng, E * I, H, 4)
    dn = layout.synth_quant(rng, E * H, I, 4)
    router = layout.f32_to_bf16(rng.normal(0, 0.02, (E, H)).astype(np.float32))
    (dg, kg), (du, ku), (dd, kd) = quant(lib, gate), quant(lib, upw), quant(lib, dn)
    rd = up(lib, router)
    out, logits = Dev(lib, H * 2, 2), Dev(lib, E * 4, 4)
    ids, wt, act = Dev(lib, TOPK * 4, 4), Dev(lib, TOPK * 2, 2), Dev(lib, TOPK * I * 2, 2)
    scratch = zeros(lib, hip.MOE_DECODE_SCRATCH_WORDS * 4, 4)
    seen = set()
    for step in range(3):
        x = layout.synth_bf16(rng, (1, H))[0]
        dx = up(lib, x)
        hip.moe_decode(rd, None, dg, du, dd, E, TOPK, dx, out, logits, ids, wt, act, scratch,
                       mode=hip.ROUTE_SOFTMAX)
        hip.check(lib.mh_stream_synchronize(None), "sync")
        want = orc.moe_decode(router, None, hip.ROUTE_SOFTMAX, gate, upw, dn, E, TOPK, H, I, x)
        assert down(lib, ids, (TOPK,), np.uint32).tolist() == want["ids"].tolist(), step
        assert np.array_equal(down(lib, logits, (E,), np.float32), want["logits"]), step
        assert np.array_equal(down(lib, wt, (TOPK,), np.uint16), want["w"]), step
        assert np.array_equal(down(lib, act, (TOPK, I), np.uint16), want["act"]), step
        assert np.array_equal(down(lib, out, (H,), np.uint16), want["out"]), step
        seen.add(tuple(want["ids"].tolist()))
        dx.free()
    for d in kg + ku + kd + [rd, out, logits, ids, wt, act, scratch]:
        d.free()
    print(f"OK config3 moe decode step, 3 steps, {len(seen)} routings", flush=True)


def main() -> None:
    lib = hip.load()
    runtimes = hip.hip_runtimes()
    assert len(runtimes) == 1 and "torch" not in runtimes[0], runtimes
    rng = np.random.default_rng(2026)
    heads(lib, rng)
    moe_decode(lib, rng)
    print(f"OK runtime {runtimes[0]}", flush=True)


if __name__ == "__main__":
    main()
