"""mh_gemv_quant_argmax_noalloc (the library's own per-device finisher
scratch, no device allocation) against mh_gemv_quant_argmax with a caller
scratch: the same logits bit for bit at batch 1 (both run the chunk-order
kernel) and within the matrix-core kernel's bound at batch 8 (both run it:
identical bits too), the same ids, on two calls in a row, the second with a
smaller input, and the oracle's ids."""
import numpy as np
import pytest

from molten_amd import hip, layout
from tests.devutil import dev_quant, empty_dev, from_dev, to_dev, zeros_dev

pytestmark = pytest.mark.gpu


def _run_pair(orc, rng, n, k, bits, batch):
    h = layout.synth_quant(rng, n, k, bits)
    x = layout.synth_bf16(rng, (batch, k))
    w, keep = dev_quant(h)
    xd = to_dev(x)
    y_ref = empty_dev((batch, n), np.uint16)
    ids_ref = empty_dev((batch,), np.uint32)
    scratch = zeros_dev((hip.argmax_scratch_words(batch),), np.uint64)
    hip.gemv_quant_argmax(w, xd, y_ref, scratch, ids_ref, batch)
    y = empty_dev((batch, n), np.uint16)
    ids = empty_dev((batch,), np.uint32)
    hip.gemv_quant_argmax_noalloc(w, xd, y, ids, batch)
    got_y, want_y = from_dev(y, np.uint16), from_dev(y_ref, np.uint16)
    np.testing.assert_array_equal(got_y, want_y)
    got_ids = from_dev(ids, np.uint32).tolist()
    assert got_ids == from_dev(ids_ref, np.uint32).tolist()
    logits = orc.gemv_quant(h, x, batch)
    assert got_ids == [orc.argmax_bf16(logits[b]) for b in range(batch)]
    return got_ids


@pytest.mark.parametrize("bits,batch", [(4, 1), (6, 8)])
def test_noalloc_matches_caller_scratch(dev, orc, bits, batch):
    print(f"noalloc bits={bits} batch={batch}", flush=True)
    hip.device_status(clear=True)
    rng = np.random.default_rng(9000 + bits * 10 + batch)
    _run_pair(orc, rng, 65536 if batch == 1 else 16384, 2048, bits, batch)  # first call: full LM-head rows
    _run_pair(orc, rng, 4096, 2048, bits, batch)  # second call: a smaller matrix on the same array
    assert hip.device_status(clear=True) == 0


def test_noalloc_rejects_batch_beyond_scratch(dev):
    w = hip.QuantWeights(0x1000, 0x2000, 0x3000, 64, 2048, 64, 4)
    with pytest.raises(hip.MoltenError, match="exceeds the library's scratch"):
        hip.gemv_quant_argmax_noalloc(w, 0x4000, None, 0x5000, 9)
