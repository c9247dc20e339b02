"""The safetensors checkpoint reader (src/safetensors.rs, src/lfm.rs
load_quant) through the C ABI.  Files are written by the `safetensors`
package (its numpy writer); header parsing, the index of shards and the
error paths run on the CPU, staged reads into device memory on the GPU."""
import json
import os
import struct

import numpy as np
import pytest

from molten_amd import hip, layout

st_numpy = pytest.importorskip("safetensors.numpy")


def _write_quant(path, base, h, extra=None):
    """A Q4/Q6 matrix as the MLX checkpoint stores it: U32 codes, BF16 scales/biases
    (bf16 written as raw 2-byte words under a BF16 header entry)."""
    tensors = {f"{base}.weight": h.codes, f"{base}.scales": h.scales, f"{base}.biases": h.biases}
    if extra:
        tensors.update(extra)
    st_numpy.save_file(tensors, str(path))
    # the numpy writer labels uint16 as U16: relabel the scale/bias entries BF16
    raw = path.read_bytes()
    n = struct.unpack("<Q", raw[:8])[0]
    header = json.loads(raw[8:8 + n])
    for name, ent in header.items():
        if name.endswith((".scales", ".biases")):
            ent["dtype"] = "BF16"
    text = json.dumps(header).encode()
    text += b" " * (-len(text) % 8)
    path.write_bytes(struct.pack("<Q", len(text)) + text + raw[8 + n:])


def test_header_names_and_meta(tmp_path, rng):
    h = layout.synth_quant(rng, 96, 512, 4)
    _write_quant(tmp_path / "model.safetensors", "model.layers.0.mlp", h,
                 {"norm.weight": np.ones(7, np.float32)})
    with hip.Checkpoint(str(tmp_path)) as ck:
        assert ck.names() == sorted(["model.layers.0.mlp.weight", "model.layers.0.mlp.scales",
                                     "model.layers.0.mlp.biases", "norm.weight"])
        assert ck.meta("model.layers.0.mlp.weight") == (hip.DTYPE_U32, (96, 64), 96 * 64 * 4)
        assert ck.meta("model.layers.0.mlp.scales") == (hip.DTYPE_BF16, (96, 8), 96 * 8 * 2)
        assert ck.meta("norm.weight") == (hip.DTYPE_F32, (7,), 28)
        with pytest.raises(hip.MoltenError, match="not in checkpoint"):
            ck.meta("missing")


def test_index_of_shards(tmp_path, rng):
    a = layout.synth_quant(rng, 16, 256, 4)
    b = layout.synth_quant(rng, 32, 256, 6)
    _write_quant(tmp_path / "s1.safetensors", "a", a)
    _write_quant(tmp_path / "s2.safetensors", "b", b)
    wm = {f"a.{t}": "s1.safetensors" for t in ("weight", "scales", "biases")}
    wm.update({f"b.{t}": "s2.safetensors" for t in ("weight", "scales", "biases")})
    (tmp_path / "model.safetensors.index.json").write_text(json.dumps({"metadata": {}, "weight_map": wm}))
    with hip.Checkpoint(str(tmp_path)) as ck:
        assert len(ck.names()) == 6
        assert ck.meta("b.weight") == (hip.DTYPE_U32, (32, 48), 32 * 48 * 4)


def test_duplicate_tensor_across_shards(tmp_path, rng):
    a = layout.synth_quant(rng, 16, 256, 4)
    _write_quant(tmp_path / "s1.safetensors", "a", a)
    _write_quant(tmp_path / "s2.safetensors", "a", a)
    (tmp_path / "model.safetensors.index.json").write_text(
        json.dumps({"weight_map": {"a.weight": "s1.safetensors", "x": "s2.safetensors"}}))
    with pytest.raises(hip.MoltenError, match="multiple shards"):
        hip.Checkpoint(str(tmp_path))


@pytest.mark.parametrize("corrupt", ["truncated", "not_json", "past_end", "reversed", "inflated",
                                     "wrapping"])
def test_bad_headers(tmp_path, rng, corrupt):
    h = layout.synth_quant(rng, 16, 256, 4)
    p = tmp_path / "model.safetensors"
    _write_quant(p, "a", h)
    raw = p.read_bytes()
    n = struct.unpack("<Q", raw[:8])[0]
    header = json.loads(raw[8:8 + n])
    if corrupt == "truncated":
        p.write_bytes(raw[:8 + n // 2])
    elif corrupt == "not_json":  # the object's closing brace replaced (same length)
        hdr = raw[8:8 + n]
        i = hdr.rindex(b"}")
        p.write_bytes(raw[:8] + hdr[:i] + b"!" + hdr[i + 1:] + raw[8 + n:])
    else:
        ent = header["a.weight"]
        a, b = ent["data_offsets"]
        ent["data_offsets"] = {
            "past_end": [0, 1 << 40],
            "reversed": [b, a],
            # inside the file but more bytes than the shape holds: a read would
            # overrun a buffer sized from the shape
            "inflated": [a, b + 8],
            # b near 2^64: data + b wraps around to a small number
            "wrapping": [a, (1 << 64) - 8],
        }[corrupt]
        text = json.dumps(header).encode()
        text += b" " * (-len(text) % 8)
        p.write_bytes(struct.pack("<Q", len(text)) + text + raw[8 + n:])
    with pytest.raises(hip.MoltenError) as ei:
        hip.Checkpoint(str(tmp_path))
    assert ei.value.code == hip.MH_ERR_INVALID


def test_missing_checkpoint(tmp_path):
    with pytest.raises(hip.MoltenError, match="no model.safetensors"):
        hip.Checkpoint(str(tmp_path))


def test_load_quant_shape_checks(tmp_path, rng):
    """load_quant's checks run before any device work."""
    h = layout.synth_quant(rng, 64, 512, 4)
    _write_quant(tmp_path / "model.safetensors", "w", h)
    with hip.Checkpoint(str(tmp_path)) as ck:
        with pytest.raises(hip.MoltenError, match="expected 6-bit, found 4"):
            ck.load_quant("w", 64, 512, 6, 0x1000, 0x2000, 0x3000)
        with pytest.raises(hip.MoltenError, match="rows 64 != 65"):
            ck.load_quant("w", 65, 512, 4, 0x1000, 0x2000, 0x3000)
        with pytest.raises(hip.MoltenError, match="scales group count"):
            ck.load_quant("w", 64, 1024, 4, 0x1000, 0x2000, 0x3000)
        with pytest.raises(hip.MoltenError, match="missing v.scales"):
            ck.load_quant("v", 64, 512, 4, 0x1000, 0x2000, 0x3000)
        with pytest.raises(hip.MoltenError, match="empty matrix"):
            ck.load_quant("w", 64, 0, 4, 0x1000, 0x2000, 0x3000)
        with pytest.raises(hip.MoltenError, match="unsupported bit width"):
            ck.load_quant("w", 64, 512, 5, 0x1000, 0x2000, 0x3000)


def test_load_quant_zero_group_scales(tmp_path, rng):
    """A scales tensor whose last dimension is 0 and k = 0 are rejected
    before any arithmetic divides by them."""
    h = layout.synth_quant(rng, 64, 512, 4)
    _write_quant(tmp_path / "model.safetensors", "w", h,
                 {"z.weight": np.zeros((64, 0), np.uint32), "z.scales": np.zeros((64, 0), np.uint16),
                  "z.biases": np.zeros((64, 0), np.uint16)})
    with hip.Checkpoint(str(tmp_path)) as ck:
        with pytest.raises(hip.MoltenError) as ei:
            ck.load_quant("z", 64, 0, 4, 0x1000, 0x2000, 0x3000)
        assert ei.value.code == hip.MH_ERR_INVALID
        with pytest.raises(hip.MoltenError, match="no columns"):
            ck.load_quant("z", 64, 512, 4, 0x1000, 0x2000, 0x3000)


@pytest.mark.gpu
@pytest.mark.parametrize("bits", [4, 6])
def test_load_quant_to_device_and_gemv(dev, bits):
    """Staged reads put the exact bytes in device memory and the GEMV over the
    loaded weights equals the oracle's.  Runs tests/ckpt_worker.py in a child
    process without torch, so that the library's HIP runtime is the only one
    in the process (as in the Rust host; torch ships its own runtime)."""
    import subprocess
    import sys
    worker = os.path.join(os.path.dirname(os.path.abspath(__file__)), "ckpt_worker.py")
    r = subprocess.run([sys.executable, worker, str(bits)], capture_output=True, text=True, timeout=120)
    assert r.returncode == 0 and r.stdout.startswith("OK"), r.stdout + r.stderr


@pytest.mark.gpu
@pytest.mark.parametrize("bits", [4, 6])
def test_load_quant_in_torch_process(dev, tmp_path, rng, orc, bits):
    """The same load in a process that also runs torch: one HIP runtime is
    mapped (torch's, which the library binds to), and the staged reads, the
    pinned staging buffers and their events work there too."""
    import torch

    from tests.devutil import dev_quant, empty_dev, from_dev, to_dev

    assert len(hip.hip_runtimes()) == 1
    h = layout.synth_quant(rng, 256, 2048, bits)
    _write_quant(tmp_path / "model.safetensors", "w", h)
    codes = torch.empty(h.codes.size, dtype=torch.int32, device=dev)
    scales = torch.empty(h.scales.size, dtype=torch.int16, device=dev)
    biases = torch.empty(h.biases.size, dtype=torch.int16, device=dev)
    with hip.Checkpoint(str(tmp_path)) as ck:
        w = ck.load_quant("w", 256, 2048, bits, codes, scales, biases)
    torch.cuda.synchronize()
    assert np.array_equal(from_dev(codes, np.uint32).reshape(h.codes.shape), h.codes)
    assert np.array_equal(from_dev(scales, np.uint16).reshape(h.scales.shape), h.scales)
    assert np.array_equal(from_dev(biases, np.uint16).reshape(h.biases.shape), h.biases)
    x = layout.synth_bf16(rng, (1, 2048))
    y = empty_dev((1, 256), np.uint16)
    hip.gemv_quant(w, to_dev(x), y, 1)
    assert np.array_equal(from_dev(y, np.uint16), orc.gemv_quant(h, x, 1))
