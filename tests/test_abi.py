"""The C ABI on the CPU: the library loads, exports every declared symbol,
and rejects bad arguments before touching the GPU runtime."""
import ctypes
import os

import pytest

from molten_amd import hip


def test_library_exports_every_declared_symbol():
    lib = hip.load()
    names = hip.declared_functions()
    assert len(names) > 10
    missing = [n for n in names if not hasattr(lib, n)]
    assert missing == []
    # and the Python binding covers every one of them
    assert sorted(set(names) - set(hip._SIGNATURES)) == []


def test_one_hip_runtime():
    """The library and torch share one HIP runtime: torch's runtime carries
    the soname the library needs, and hip.load() imports torch first."""
    import torch  # noqa: F401

    hip.load()
    rts = hip.hip_runtimes()
    assert len(rts) == 1, rts
    assert "torch" in rts[0], rts


def test_ceiling_library_exports():
    """The measurement kernels' library (bench.py --ceilings) exports what
    include/molten_ceiling.h declares and rejects bad arguments on the host."""
    import os
    import re

    root = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
    text = open(os.path.join(root, "include", "molten_ceiling.h")).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    names = sorted(set(re.findall(r"\b(mhc_[a-z0-9_]+)\s*\(", text)))
    assert names == ["mhc_copy", "mhc_exchange", "mhc_lds_fill", "mhc_mfma", "mhc_mfma_flops", "mhc_read"]
    hip.load()
    lib = ctypes.CDLL(os.path.join(root, "molten_amd", "libmolten_ceiling.so"))
    for n in names:
        assert hasattr(lib, n), n
    lib.mhc_read.argtypes = [ctypes.c_void_p, ctypes.c_size_t, ctypes.c_uint32, ctypes.c_uint32,
                             ctypes.c_int, ctypes.c_void_p, ctypes.c_void_p]
    assert lib.mhc_read(0x1000, 100, 8, 1, 0, 0x2000, None) == -1   # not a multiple of 16
    assert lib.mhc_read(0x1000, 1024, 8, 3, 0, 0x2000, None) == -1  # unroll 3
    lib.mhc_exchange.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_uint32, ctypes.c_uint64, ctypes.c_int,
                                 ctypes.c_uint32, ctypes.c_uint32, ctypes.c_void_p]
    assert lib.mhc_exchange(0x1000, 0x2000, 8, 1, 0, 100, 16, None) == -1     # no consumer workgroups
    assert lib.mhc_exchange(0x1000, 0x2000, 256, 1, 2, 100, 16, None) == -1   # mode 2
    assert lib.mhc_exchange(0x1004, 0x2000, 256, 1, 0, 100, 16, None) == -1   # words not 8-byte aligned
    assert lib.mhc_exchange(0x1000, 0x2000, 256, 1, 0, 100, 0, None) == -1    # no polls
    lib.mhc_lds_fill.argtypes = [ctypes.c_uint32, ctypes.c_uint32, ctypes.c_void_p]
    assert lib.mhc_lds_fill(0, 0, None) == -1  # no workgroups
    lib.mhc_mfma_flops.restype = ctypes.c_uint64
    assert lib.mhc_mfma_flops(2, 3) == 2 * 4 * 3 * 8 * 32 * 32 * 16 * 2


def test_version():
    assert b"gfx950" in hip.load().mh_version()


def _qw(**kw):
    base = dict(codes=0x1000, scales=0x2000, biases=0x3000, out_features=64, in_features=2048,
                group_size=64, bits=4)
    base.update(kw)
    return hip.QuantWeights(base["codes"], base["scales"], base["biases"], base["out_features"],
                            base["in_features"], base["group_size"], base["bits"])


@pytest.mark.parametrize("kw,code", [
    (dict(bits=3), hip.MH_ERR_UNSUPPORTED),
    (dict(bits=8), hip.MH_ERR_UNSUPPORTED),  # the GEMVs read 4- and 6-bit codes only
    (dict(group_size=48), hip.MH_ERR_UNSUPPORTED),
    (dict(in_features=2000), hip.MH_ERR_INVALID),
    (dict(out_features=0), hip.MH_ERR_INVALID),
    (dict(codes=0x1008), hip.MH_ERR_ALIGN),
    (dict(codes=None), hip.MH_ERR_INVALID),
])
def test_gemv_rejects_bad_weights(kw, code):
    with pytest.raises(hip.MoltenError) as ei:
        hip.gemv_quant(_qw(**kw), 0x4000, 0x5000, stream=0)
    assert ei.value.code == code
    assert hip.load().mh_last_error()  # message set


def test_gemv_rejects_bad_batch_and_pointers():
    for batch in (0, 9):
        with pytest.raises(hip.MoltenError) as ei:
            hip.gemv_quant(_qw(), 0x4000, 0x5000, batch=batch, stream=0)
        assert ei.value.code == hip.MH_ERR_UNSUPPORTED
    with pytest.raises(hip.MoltenError):
        hip.gemv_quant(_qw(), None, 0x5000, stream=0)
    with pytest.raises(hip.MoltenError):
        hip.gemv_quant(_qw(), 0x4000, None, stream=0)
    # Q6 codes need 8-byte alignment only
    with pytest.raises(hip.MoltenError) as ei:
        hip.gemv_quant(_qw(bits=6, codes=0x1004), 0x4000, 0x5000, stream=0)
    assert ei.value.code == hip.MH_ERR_ALIGN


def test_argmax_arguments():
    with pytest.raises(hip.MoltenError):
        hip.gemv_head_argmax(_qw(), 0x4000, None, stream=0)
    with pytest.raises(hip.MoltenError) as ei:
        hip.gemv_quant_argmax(_qw(), 0x4000, 0x5000, 0x6004, 0x7000, stream=0)
    assert ei.value.code == hip.MH_ERR_ALIGN
    with pytest.raises(hip.MoltenError):  # scratch without ids
        hip.gemv_quant_argmax(_qw(), 0x4000, 0x5000, 0x6000, None, stream=0)
    with pytest.raises(hip.MoltenError):  # no stamp buffer
        hip.gemv_quant_argmax_stamped(_qw(), 0x4000, 0x5000, 0x6000, 0x7000, None, stream=0)
    with pytest.raises(hip.MoltenError):  # stamps not 8-byte aligned
        hip.gemv_quant_argmax_stamped(_qw(), 0x4000, 0x5000, 0x6000, 0x7000, 0x8004, stream=0)
    with pytest.raises(hip.MoltenError) as ei:  # a batch without a stamped kernel
        hip.gemv_quant_argmax_stamped(_qw(), 0x4000, 0x5000, 0x6000, 0x7000, 0x8000, batch=3, stream=0)
    assert ei.value.code == hip.MH_ERR_UNSUPPORTED
    with pytest.raises(hip.MoltenError):
        hip.token_tail(0x6000, 0x7000, batch=0, stream=0)
    with pytest.raises(hip.MoltenError):
        hip.argmax_bf16(0x4000, 0, 0x6000, 0x7000, stream=0)


def test_bulk_dequant_needs_k_multiple_of_128():
    with pytest.raises(hip.MoltenError):
        hip.dequant_q4_bf16_bulk(_qw(in_features=64 * 3), 0x8000, stream=0)
    with pytest.raises(hip.MoltenError):
        hip.dequant_q4_bf16_bulk(_qw(bits=6), 0x8000, stream=0)


def test_memcpy_kind_checked():
    lib = hip.load()
    assert lib.mh_memcpy(None, None, 0, 7, None) == hip.MH_ERR_INVALID


def test_proj3_and_conv3_arguments():
    q = _qw(out_features=64)
    with pytest.raises(hip.MoltenError) as ei:  # pos beyond the cache
        hip.proj3_gemv_scatter(q, q, q, 0x4000, 0x5000, 0x6000, 0x7000, 8, 8, stream=0)
    assert ei.value.code == hip.MH_ERR_INVALID
    with pytest.raises(hip.MoltenError) as ei:  # V rows not whole heads
        hip.proj3_gemv_scatter(q, q, _qw(out_features=96), 0x4000, 0x5000, 0x6000, 0x7000, 8, 0,
                               stream=0)
    assert ei.value.code == hip.MH_ERR_INVALID
    with pytest.raises(hip.MoltenError) as ei:  # the reference's projections are 4-bit
        hip.proj3_gemv_scatter(q, _qw(bits=6), q, 0x4000, 0x5000, 0x6000, 0x7000, 8, 0, stream=0)
    assert ei.value.code == hip.MH_ERR_UNSUPPORTED
    with pytest.raises(hip.MoltenError) as ei:  # 3H rows
        hip.conv3_gemv(_qw(out_features=64), 0x4000, 0x5000, 0x6000, 0x7000, 0x8000, stream=0)
    assert ei.value.code == hip.MH_ERR_INVALID
    with pytest.raises(hip.MoltenError) as ei:
        hip.conv3_gemv(_qw(out_features=48, in_features=4096), 0x4000, 0x5000, 0x6000, 0x7000,
                       0x8000, stream=0)
    assert ei.value.code == hip.MH_ERR_UNSUPPORTED


def test_embedding_arguments():
    with pytest.raises(hip.MoltenError) as ei:  # the table is 6-bit
        hip.gather_rows_q6(_qw(), 0x4000, 4, 0x5000, stream=0)
    assert ei.value.code == hip.MH_ERR_UNSUPPORTED
    with pytest.raises(hip.MoltenError) as ei:
        hip.gather_rows_q6(_qw(bits=6), 0x4000, 4, 0x5008, stream=0)
    assert ei.value.code == hip.MH_ERR_ALIGN
    with pytest.raises(hip.MoltenError) as ei:
        hip.gather_rows_q6(_qw(bits=6), 0x4000, 0, 0x5000, stream=0)
    assert ei.value.code == hip.MH_ERR_INVALID
    with pytest.raises(hip.MoltenError) as ei:
        hip.token_tail_embed(0x6000, 0x7000, _qw(bits=6, in_features=4096), 0x4000, 0x5000, 0x8000,
                             1e-5, stream=0)
    assert ei.value.code == hip.MH_ERR_UNSUPPORTED
    with pytest.raises(hip.MoltenError) as ei:
        hip.token_tail_embed(0x6000, 0x7000, _qw(bits=6), 0x4008, 0x5000, 0x8000, 1e-5, stream=0)
    assert ei.value.code == hip.MH_ERR_ALIGN


def test_dense_gemm_arguments():
    with pytest.raises(hip.MoltenError) as ei:
        hip.gemm_q4_dense(0x4000, 16, _qw(bits=6), 0x5000, stream=0)
    assert ei.value.code == hip.MH_ERR_UNSUPPORTED
    with pytest.raises(hip.MoltenError) as ei:
        hip.gemm_q4_dense(0x4008, 16, _qw(), 0x5000, stream=0)
    assert ei.value.code == hip.MH_ERR_ALIGN
    with pytest.raises(hip.MoltenError) as ei:
        hip.gemm_q4_dense(0x4000, 0, _qw(), 0x5000, stream=0)
    assert ei.value.code == hip.MH_ERR_INVALID


def test_bf16_and_quant_gemm_arguments():
    with pytest.raises(hip.MoltenError) as ei:
        hip.gemm_bf16_nt(None, 0x5000, 0x6000, 4, 4, 64, stream=0)
    assert ei.value.code == hip.MH_ERR_INVALID
    with pytest.raises(hip.MoltenError) as ei:
        hip.gemm_bf16_nt(0x4001, 0x5000, 0x6000, 4, 4, 64, stream=0)
    assert ei.value.code == hip.MH_ERR_ALIGN
    hip.gemm_bf16_nt(0x4000, 0x5000, 0x6000, 0, 4, 64, stream=0)  # M = 0: nothing to do
    with pytest.raises(hip.MoltenError, match="dequant scratch holds 100 bf16 elements, needs 131072"):
        hip.gemm_quant_bf16_nt(0x4000, 8, _qw(), 0x6000, 0x7000, 100, stream=0)
    with pytest.raises(hip.MoltenError) as ei:
        hip.gemm_quant_bf16_nt(0x4000, 8, _qw(bits=3), 0x6000, 0x7000, 1 << 20, stream=0)
    assert ei.value.code == hip.MH_ERR_UNSUPPORTED
    with pytest.raises(hip.MoltenError) as ei:
        hip.gemm_quant_bf16_nt(0x4000, 8, _qw(bits=8), 0x6000, 0x7008, 1 << 20, stream=0)
    assert ei.value.code == hip.MH_ERR_ALIGN
    with pytest.raises(hip.MoltenError) as ei:  # 8-bit codes are read 16 bytes at a time
        hip.dequant_to_bf16(_qw(bits=8, codes=0x1008), 0x6000, stream=0)
    assert ei.value.code == hip.MH_ERR_ALIGN


def test_grouped_gemm_rejects_operands_past_4_gib():
    """The tile kernel forms A and weight offsets in 32 bits: operands of 4 GiB
    or more are refused on the host (no device call is made)."""
    with pytest.raises(hip.MoltenError, match="exceed 4 GiB") as ei:
        hip.gemm_q4_dense(0x4000, 1 << 20, _qw(out_features=256), 0x6000, stream=0)  # A = 4 GiB
    assert ei.value.code == hip.MH_ERR_UNSUPPORTED
    with pytest.raises(hip.MoltenError, match="exceed 4 GiB") as ei:  # weights = 4 GiB
        hip.gemm_q4_dense(0x4000, 64, _qw(out_features=1 << 22), 0x6000, stream=0)
    assert ei.value.code == hip.MH_ERR_UNSUPPORTED
    with pytest.raises(hip.MoltenError, match="exceed 4 GiB") as ei:  # gathered rows, grouped map
        hip.gemm_q4_grouped_mlx(0x4000, _qw(out_features=256), 0x6000, 0x7000, 8, 1 << 20, 256,
                                hip.MoeTile.T128, stream=0)
    assert ei.value.code == hip.MH_ERR_UNSUPPORTED


def test_ordered_grouped_gemm_arguments():
    """The launch-ordered grouped GEMMs take whole 8 x (n / bn) units of
    entries, segment tile widths only and (gate/up) the row gather; all
    refused on the host."""
    w = _qw(out_features=512)
    with pytest.raises(hip.MoltenError, match="whole units") as ei:  # nt = 2: units of 16
        hip.gemm_q4_grouped_ordered(0x4000, w, 0x6000, 0x7000, 24, 64, 512, hip.MoeTile.DN512, stream=0)
    assert ei.value.code == hip.MH_ERR_INVALID
    with pytest.raises(hip.MoltenError) as ei:
        hip.gemm_q4_grouped_ordered(0x4000, w, 0x6000, 0x7000, 32, 64, 512, (512, 128), stream=0)
    assert ei.value.code == hip.MH_ERR_UNSUPPORTED
    with pytest.raises(hip.MoltenError) as ei:
        hip.gemm_q4_grouped_gu_act_ordered(0x4000, None, 64, w, w, 0x6000, 0x7000, 32, 64, 256,
                                           hip.MoeTile.GU512, stream=0)
    assert ei.value.code == hip.MH_ERR_INVALID
    with pytest.raises(hip.MoltenError) as ei:
        hip.gemm_q4_grouped_gu_act_ordered(0x4000, 0x5000, 64, w, w, 0x6000, 0x7000, 32, 64, 256,
                                           (512, 256), stream=0)
    assert ei.value.code == hip.MH_ERR_UNSUPPORTED
    assert hip.map_grid(1152, 12) == 1152 and hip.map_grid(1153, 12) == 1248 and hip.map_grid(1, 8) == 64


def test_sample_draw_arguments():
    p = hip.sample_params(1.0, 1, 0, top_k=40)
    with pytest.raises(hip.MoltenError, match="workspace holds 16 bytes"):
        hip.sample_draw(0x4000, 128000, None, p, 0x6000, 0x7000, 16, stream=0)
    with pytest.raises(hip.MoltenError) as ei:
        hip.sample_draw(0x4000, 128000, None, hip.sample_params(1.0, 1, 0, top_p=0.0), 0x6000, 0x7000,
                        1 << 20, stream=0)
    assert ei.value.code == hip.MH_ERR_INVALID
    with pytest.raises(hip.MoltenError) as ei:
        hip.sample_draw(0x4000, 128000, None, p, 0x6000, 0x7010, 1 << 20, stream=0)
    assert ei.value.code == hip.MH_ERR_ALIGN
    assert hip.sample_workspace_bytes(128000) >= 128000 * 4


def test_sample_arguments():
    p = hip.sample_params(1.0, 1, 0)
    with pytest.raises(hip.MoltenError) as ei:
        hip.sample_gumbel(0x4000, 128000, 0x5000, hip.sample_params(1.0, 1, 0, top_k=40), 0x6000, stream=0)
    assert ei.value.code == hip.MH_ERR_UNSUPPORTED
    with pytest.raises(hip.MoltenError) as ei:
        hip.sample_gumbel(0x4000, 128002, 0x5000, p, 0x6000, stream=0)
    assert ei.value.code == hip.MH_ERR_INVALID
    with pytest.raises(hip.MoltenError) as ei:  # the penalty reads the seen set
        hip.sample_gumbel(0x4000, 128000, None, hip.sample_params(1.0, 1, 0, penalty=1.2), 0x6000, stream=0)
    assert ei.value.code == hip.MH_ERR_INVALID


def test_python_mirrors_of_header_constants():
    """The sizes hip.py hands to callers match the header's defines."""
    import re
    text = open(os.path.join(os.path.dirname(__file__), "..", "include", "molten_hip.h")).read()

    def define(name):
        m = re.search(r"#define %s (\d+)u" % name, text)
        assert m, name
        return int(m.group(1))

    assert hip.SAMPLE_ZERO_BYTES == define("MH_SAMPLE_ZERO_BYTES")
    assert hip.ARGMAX_SLOTS == define("MH_ARGMAX_SLOTS")
    assert hip.MOE_DECODE_SCRATCH_WORDS == define("MH_MOE_DECODE_SCRATCH_WORDS")
    assert hip.MOE_DECODE_STAMP_WAVES == define("MH_MOE_DECODE_STAMP_WAVES")
    assert hip.MOE_DECODE_STAMPS == define("MH_MOE_DECODE_STAMPS")
    assert hip.GEMV_STAMP_WAVES == define("MH_GEMV_STAMP_WAVES")
    assert hip.GEMV_STAMPS == define("MH_GEMV_STAMPS")
    assert hip.PREFILL_STAMP_WGS == define("MH_PREFILL_STAMP_WGS")
    assert hip.PREFILL_STAMPS == define("MH_PREFILL_STAMPS")
    # the workspace regions, in the header's enum order
    enum = re.search(r"enum \{\s*(MH_PREFILL_WS_LOGITS[^}]*)\}", text).group(1)
    names = [w.strip().split("=")[0].strip() for w in enum.split(",") if w.strip()]
    assert names[-1] == "MH_PREFILL_WS_REGIONS"
    assert [n[len("MH_PREFILL_WS_"):].lower() for n in names[:-1]] == hip.PREFILL_WS_REGIONS
