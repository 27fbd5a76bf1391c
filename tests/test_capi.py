"""The C-ABI library loads without a GPU, exports every entry point declared in
include/ecdecode.h, and rejects bad arguments on the host before any launch."""
import ctypes
import re
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parent.parent
HEADER = ROOT / "include" / "ecdecode.h"



# ecd_sample_topk_next without the folded attention: qkv .. HD, stream
_NOATT = (None, 0, 0, None, None, 0, 0, None, 0, 0, 0, 0, None, 0, None, 0, None)

def declared():
    text = HEADER.read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return re.findall(r"\b(ecd_\w+)\s*\(", text)


def test_header_declares_entry_points():
    names = declared()
    assert "ecd_gemv_i8" in names and "ecd_decode_attn" in names
    assert len(names) == len(set(names))


def test_library_exports_every_declared_symbol():
    from estudiocanciones_amd import _ffi
    lib = _ffi.lib()
    for name in declared():
        assert hasattr(lib, name), f"{name} declared in ecdecode.h but not exported"
    # and the binding declares exactly the same entry points
    assert set(_ffi.SIGNATURES) | {"ecd_version"} == set(declared())
    assert lib.ecd_version().startswith(b"ecdecode")


def test_signatures_match_header_arity():
    from estudiocanciones_amd import _ffi
    text = re.sub(r"/\*.*?\*/", "", HEADER.read_text(), flags=re.S)
    for name, argtypes in _ffi.SIGNATURES.items():
        m = re.search(name + r"\s*\(([^)]*)\)", text)
        assert m, name
        nargs = len([a for a in m.group(1).split(",") if a.strip()])
        assert nargs == len(argtypes), f"{name}: header has {nargs} args, binding {len(argtypes)}"


def _taps(*offsets):
    return (ctypes.c_int * len(offsets))(*offsets)


@pytest.mark.parametrize("call", [
    lambda L: L.ecd_gemv_i8(None, 64, None, None, None, 0, None, 64, 1, 64, 64, 0, None),
    lambda L: L.ecd_gemv_i8(8, 32, 8, 8, None, 0, 8, 64, 1, 64, 64, 0, None),     # ldx < K
    lambda L: L.ecd_gemv_i8(8, 64, 8, 8, None, 0, 8, 64, 0, 64, 64, 0, None),     # M = 0
    lambda L: L.ecd_rmsnorm(None, 8, None, None, 8, 1, 8, 1e-5, None),
    lambda L: L.ecd_rope_kv_write(8, 8, 8, 8, 8, 8, 1, 1, 3, 2, 8, 128, None),    # Hq % Hk
    lambda L: L.ecd_rope_kv_write(8, 8, 8, 8, 8, 8, 1, 1, 4, 2, 8, 127, None),    # odd HD
    lambda L: L.ecd_decode_attn(8, 8, 8, 8, 8, None, None, None, 1, 1, 8, 2, 8, 128, 16, 0.1, None),
    lambda L: L.ecd_decode_attn(8, 8, 8, 8, None, None, None, None, 1, 1, 8, 2, 8, 128, 1, 0.1, None),
    lambda L: L.ecd_attn_combine(None, None, None, None, 1, 128, 16, None),
    lambda L: L.ecd_decode_attn_noalloc(8, 8, 8, 8, None, 1, 1, 8, 2, 8, 128, 16, 0.1, None),   # no o
    lambda L: L.ecd_decode_attn_noalloc(8, 8, 8, 8, 8, 1, 1, 8, 3, 8, 128, 16, 0.1, None),      # Hq % Hk
    lambda L: L.ecd_decode_attn_merged(8, 8, 8, 8, 8, 8, None, 1, 1, 24, 8, 4096, 128, 4, 0.1, None),  # no cnt
    lambda L: L.ecd_decode_attn_merged(8, 8, 8, 8, 8, 8, 8, 1, 1, 24, 8, 4096, 128, 0, 0.1, None),     # kb 0
    lambda L: L.ecd_decode_attn_merged(8, 8, 8, 8, 8, 8, 8, 1, 1, 24, 8, 4096, 128, 33, 0.1, None),    # kb 33
    lambda L: L.ecd_decode_attn_merged(8, 8, 8, 8, 8, 8, 8, 1, 1, 24, 7, 4096, 128, 4, 0.1, None),     # Hq % Hk
    lambda L: L.ecd_gemv_i8p_splitk(16, 64, 16, 16, None, 0, 16, 64, 1, 64, 192, 2, 16, 0, None),  # 3 chunks % 2
    lambda L: L.ecd_silu_mul(8, 8, 0, 8192, None),
    lambda L: L.ecd_sample_topk_next(16, 8256, 8, 4, 1.5, 1.0, 50, 8197, 16, None, None, 0, 16, 1,
                                     16, 1024, 8196, 16, 1024, 1024, *_NOATT),   # rows_n < V
    lambda L: L.ecd_sample_topk_next(16, 8256, 8, 4, 1.5, 1.0, 50, 8197, 16, None, None, 0, 16, 1,
                                     16, 1024, 8197, 16, 1024, 1020, *_NOATT),   # D % 8
    lambda L: L.ecd_sample_topk_next(16, 8256, 8, 4, 1.5, 1.0, 50, 8197, 16, None, None, 0, 16, 1,
                                     24, 1024, 8197, 16, 1024, 1024, *_NOATT),   # rows not 16-aligned
    lambda L: L.ecd_sample_topk_next(16, 8256, 8, 4, 1.5, 1.0, 50, 8197, 16, None, None, 0, 16, 1,
                                     16, 1024, 8197, None, 1024, 1024, *_NOATT), # no x
    lambda L: L.ecd_sample_topk_next(16, 8256, 8, 3, 1.5, 1.0, 50, 8197, 16, None, None, 0, 16, 1,
                                     16, 1024, 8197, 16, 1024, 1024, *_NOATT),   # B != N, 2N
    lambda L: L.ecd_sample_topk_next(16, 8256, 8, 4, 1.5, 1.0, 50, 8197, 16, None, None, 0, 16, 1,
                                     16, 1024, 8197, 16, 1024, 1024, 16, 1536, 8197, 16, 16, 8, 8,
                                     16, 1024, 8, 2, 128, None, 0, None, 0, None),  # p = L
    lambda L: L.ecd_sample_topk_next(16, 8256, 8, 4, 1.5, 1.0, 50, 8197, 16, None, None, 0, 16, 1,
                                     16, 1024, 8197, 16, 1024, 1024, 16, 2048, 8197, 16, 16, 8, 3,
                                     16, 1536, 12, 2, 128, None, 0, None, 0, None),  # G = 6 > 4
    lambda L: L.ecd_sample_topk_next(16, 8256, 8, 4, 1.5, 1.0, 50, 8197, 16, None, None, 0, 16, 1,
                                     16, 1024, 8197, 16, 1024, 1024, 16, 2048, 8197, 16, 16, 8, 3,
                                     16, 1024, 8, 4, 128, None, 0, None, 0, None),  # 2 x 4 pairs
    lambda L: L.ecd_sample_topk_next(16, 8256, 8, 4, 1.5, 1.0, 50, 8197, 16, None, None, 0, 16, 1,
                                     16, 1024, 8197, 16, 1024, 1024, 16, 1536, 8197, None, 16, 8,
                                     3, 16, 1024, 8, 2, 128, None, 0, None, 0, None),  # no k cache
    lambda L: L.ecd_sample_topk_next(16, 8256, 8, 4, 1.5, 1.0, 50, 8197, 16, None, None, 0, 16, 1,
                                     16, 1024, 8197, 16, 1024, 1024, None, 0, 0, None, None, 0, 0,
                                     None, 0, 0, 0, 0, 16, 1024, None, 1024, None),  # ev without xe
    lambda L: L.ecd_sample_topk_next(16, 8256, 8, 4, 1.5, 1.0, 50, 8197, 16, None, None, 0, 16, 1,
                                     16, 3072, 8197, 16, 3072, 3072, 16, 4096, 8197, 16, 16, 8, 3,
                                     16, 2048, 8, 4, 256, None, 0, None, 0, None),  # head_dim 256
    lambda L: L.ecd_sample_topk_next(16, 8256, 8, 4, 1.5, 1.0, 50, 8197, 16, None, None, 0, 16, 1,
                                     16, 3072, 8197, 16, 3072, 3072, 16, 6144, 8197, 16, 16, 16, 8,
                                     16, 3072, 8, 4, 384, None, 0, None, 0, None),  # 384: p = 8
    lambda L: L.ecd_sample_topk_next(16, 8256, 8, 4, 1.5, 1.0, 50, 8197, 16, None, None, 0, 16, 1,
                                     16, 3072, 8197, 16, 3072, 3072, 16, 12288, 8197, 16, 16, 8, 3,
                                     16, 3072, 8, 8, 384, None, 0, None, 0, None),  # 384: 2 x 8 pairs
    lambda L: L.ecd_sample_topk_next(16, 8256, 8, 4, 1.5, 1.0, 50, 8197, 16, None, None, 0, 16, 1,
                                     16, 3072, 8197, 16, 3072, 3072, 16, 4608, 8197, 16, 16, 8, 3,
                                     16, 1536, 4, 4, 384, None, 0, None, 0, None),  # 384: G = 1
    lambda L: L.ecd_sample_topk_next(16, 8256, 8, 4, 1.5, 1.0, 50, 8197, 16, None, None, 0, 16, 1,
                                     16, 4096, 8197, 16, 4096, 4096, *_NOATT),      # D > 3072
    lambda L: L.ecd_embed_sum_i8(None, 8, 8, 65576, 8, 1, 8, 8, 8197, None),
    lambda L: L.ecd_embed_i8(8, 0, 8, 8, 65576, 0, 8197, None, 8, 1, 8, None),    # stride 0
    lambda L: L.ecd_embed_i8(8, 1, 8, 8, 0, 0, 8197, None, 8, 1, 8, None),        # rows 0
    lambda L: L.ecd_quantize_rows_i8(8, 8, None, None, 1, 8, None),               # no scale out
    lambda L: L.ecd_rope_table(None, 8, 128, 5e5, 32.0, 1.0, 4.0, 8192.0, None),
    lambda L: L.ecd_rope_table(8, 8, 127, 5e5, 32.0, 1.0, 4.0, 8192.0, None),
    lambda L: L.ecd_copy_bytes(8, 8, 15, None),
    lambda L: L.ecd_frame_advance(8, 8, 8, 8, 8, 1, 8, 8, 65, 4, 10, 60, 8193, None),  # B > 64
    lambda L: L.ecd_frame_advance(8, 8, 8, 8, 8, 1, 8, 8, 8, 9, 10, 60, 8193, None),   # N > B
    lambda L: L.ecd_frame_advance(8, 4, 8, 8, 8, 1, 8, 8, 8, 4, 10, 60, 8193, None),   # lds < 8
    lambda L: L.ecd_prefill_attn(16, 16, 16, 16, 16, 1, 8, 24, 8, 64, 96, 0.1, None),    # HD 96
    lambda L: L.ecd_prefill_attn(16, 16, 16, 16, 16, 1, 8, 40, 8, 64, 128, 0.1, None),   # G = 5
    lambda L: L.ecd_prefill_attn(18, 16, 16, 16, 16, 1, 8, 24, 8, 64, 128, 0.1, None),   # q align
    lambda L: L.ecd_prefill_attn(16, 16, 16, 16, 16, 1, 8, 24, 8, 64, 128, 0.0, None),   # scale <= 0
    lambda L: L.ecd_codec_rope_table(16, 8, 63, None),                             # odd HD
    lambda L: L.ecd_codec_rope_heads(16, 192, 16, 16, 16, 16, 1, 8, 1, 60, None),   # HD % 8
    lambda L: L.ecd_codec_rope_heads(16, 100, 16, 16, 16, 16, 1, 8, 1, 64, None),   # ldq < 3D
    lambda L: L.ecd_codec_norm_mod(16, None, None, None, 0, 16, 16, 16, 16, 16, 0, 16, 8, 8,
                                   8200, 0, 1e-6, None),                            # D > 4096
    lambda L: L.ecd_codec_norm_mod(16, 16, None, None, 0, 16, 16, 16, 16, 16, 0, 16, 8, 8, 64,
                                   0, 1e-6, None),                                  # h, no gate
    lambda L: L.ecd_codec_norm_mod(16, None, None, None, 0, None, 16, 16, 16, 16, 0, 16, 8, 8,
                                   64, 0, 1e-6, None),                              # RMS, no w
    lambda L: L.ecd_codec_cols3(None, None, None, None, None, None, 1, 16, 1, 8, None),
    lambda L: L.ecd_codec_vq_embed(16, 8, 1, 16, 16, 1, 8, 10, 8192, 30, 64, 0, None),  # Dc % 8
    lambda L: L.ecd_codec_vq_embed(16, 8, 1, 16, 16, 1, 8, 10, 8192, 32, 24, 0, None),  # Wp < Dc
    lambda L: L.ecd_codec_vq_embed(16, 8, 1, 16, 16, 1, 8, 10, 8192, 32, 64, 2, None),  # clamp 2
    lambda L: L.ecd_codec_timestep(None, 16, 1, None),
    lambda L: L.ecd_codec_silu(16, 16, 0, None),
    lambda L: L.ecd_codec_euler(16, 16, 16, 16, 2, 1, 8, 256, 0, 0.1, 1.2, 0.0, 0, None),  # cfg 2
    lambda L: L.ecd_codec_euler(16, None, 16, 16, 1, 1, 8, 256, 4, 0.1, 1.2, 0.0, 0, None),  # blend, no noise
    lambda L: L.ecd_codec_euler(16, 16, 16, 16, 1, 1, 8, 252, 0, 0.1, 1.2, 0.0, 0, None),  # C % 8
    lambda L: L.ecd_codec_cols_taps(16, 64, _taps(0, -1), 2, 16, 1, 8, 64, 1, 0, 0, 9, None),  # rows > B*T
    lambda L: L.ecd_gemm_f16p_conv(16, 64, 16, None, 1.0, None, 0, 16, 64, 100, 64, 128, 30, 60, -1,
                                   _taps(0, -1), 2, 1, 0, None),                    # M % T
    lambda L: L.ecd_gemm_f16p_conv(16, 64, 16, None, 1.0, None, 0, 16, 64, 90, 64, 128, 30, 60, -1,
                                   _taps(-61, 0), 2, 1, 0, None),                   # tap beyond the pad
    lambda L: L.ecd_gemm_f16p_conv(16, 64, 16, None, 1.0, None, 0, 16, 64, 90, 64, 192, 30, 60, -1,
                                   _taps(0, -1), 2, 1, 0, None),                    # K % (64 k)
    lambda L: L.ecd_gemm_f16p_conv(16, 64, 16, None, 1.0, None, 0, 16, 64, 90, 64, 128, 30, 60, -1,
                                   _taps(0, -1), 2, 1, 1, None),                    # no SiLU epilogue
    lambda L: L.ecd_gemm_f16p_conv(16, 64, 16, None, 1.0, None, 0, 16, 64, 90, 64, 128, 30, 60, -1,
                                   None, 2, 1, 0, None),                         # taps missing
    lambda L: L.ecd_gemm_f16p_conv(16, 64, 16, None, 1.0, None, 0, 16, 64, 90, 64, 128, 30, 60, -1,
                                   _taps(0, -1), 2, 3, 0, None),                 # rep 3
    lambda L: L.ecd_gemm_f16p_conv(16, 64, 16, None, 1.0, None, 0, 16, 64, 93, 64, 128, 31, 60, -1,
                                   _taps(0, -1), 2, 2, 0, None),                 # rep 2, odd T
    lambda L: L.ecd_gemm_f16p_conv(16, 64, 16, None, 1.0, None, 0, 16, 64, 90, 64, 128, 30, 4, -1,
                                   _taps(-10, 0), 2, 2, 0, None),                # rep 2, tap past pad
    lambda L: L.ecd_gemm_f16p_rope(16, 64, 16, None, 16, 16, 16, 16, 90, 30, 2, 62, 64, None),  # HD % 4
    lambda L: L.ecd_gemm_f16p_rope(16, 64, 16, None, 16, 16, 16, 16, 100, 30, 2, 64, 64, None),  # M % T
    lambda L: L.ecd_gemm_f16p_rope(16, 64, 16, None, 16, 16, 12, 16, 90, 30, 2, 64, 64, None),  # k align
    lambda L: L.ecd_layer_tail(*([256] * 24), 17, 3072, 8192, 1, 24, 8, 1024, 128, 1e-5, 0,
                               None),                                           # M > 16
    lambda L: L.ecd_layer_tail(*([256] * 22), None, 256, 8, 3072, 8192, 1, 24, 8, 1024, 128, 1e-5,
                               0, None),                                        # no err word
    lambda L: L.ecd_layer_tail(*([256] * 21), 16, 256, 256, 8, 3072, 8192, 1, 24, 8, 1024, 128,
                               1e-5, 0, None),                                  # sync not 256-aligned
    lambda L: L.ecd_layer_tail(*([256] * 24), 8, 3072, 8192, 1, 24, 7, 1024, 128, 1e-5, 0,
                               None),                                           # Hq % Hk
    lambda L: L.ecd_layer_tail(*([256] * 10), None, *([256] * 6), 256, *([256] * 6), 8, 3072,
                               8192, 1, 24, 8, 1024, 128, 1e-5, 0, None),       # o_next, no wq
])
def test_host_argument_validation(call):
    """Invalid arguments return ECD_EINVAL before any HIP call (no GPU needed)."""
    from estudiocanciones_amd import _ffi
    assert call(_ffi.lib()) == _ffi.ECD_EINVAL


def _stack_records(nl, M=8, D=3072, F=8192, HD=384, Hq=8):
    """Host layer records of ecd_layer_stack_plan with fake, disjoint, aligned addresses."""
    import numpy as np
    rec = np.zeros((nl, 17), np.uint64)
    base = 1 << 32
    for i in range(nl):
        rec[i, :12] = 256                                # weights, norms, caches: any aligned
        rec[i, 12] = base + i * (1 << 24)                # x1
        rec[i, 13] = base + i * (1 << 24) + (1 << 20)    # mm
        rec[i, 14] = base + i * (1 << 24) + (2 << 20)    # xout
        rec[i, 15] = base + i * (1 << 24) + (3 << 20)    # o_next
    rec[nl - 1, 7:12] = 0                                # the last layer: no next layer
    rec[nl - 1, 15] = 0
    return rec


@pytest.mark.parametrize("case", ["nl0", "mid_no_next", "last_o_next_without_wq", "overlap",
                                  "cross_layer_overlap", "misaligned", "plan_misaligned",
                                  "head_not_last", "head_3072_wide", "head_with_cache",
                                  "head_overlaps"])
def test_layer_stack_plan_rejects_bad_records(case):
    """ecd_layer_stack_plan checks every record on the host before copying the plan: a middle
    layer without the next layer's q|k|v and attention, outputs that overlap (within a layer or
    across layers), unaligned buffers; and ecd_layer_stack rejects a bad layer count."""
    from estudiocanciones_amd import _ffi
    L = _ffi.lib()
    nl = 3
    rec = _stack_records(nl)
    plan = 4096
    if case == "nl0":
        assert L.ecd_layer_stack(plan, 0, 256, 256, 256, 256, 256, 256, 256, 256, 8, 3072, 8192,
                                 1, 8, 4, 8, 384, 0, 0, 1e-5, 0, None) == _ffi.ECD_EINVAL
        return
    if case == "mid_no_next":
        rec[1, 8] = 0                        # wq of a middle layer
    elif case == "last_o_next_without_wq":
        rec[nl - 1, 15] = rec[nl - 1, 14] + (1 << 16)
    elif case == "overlap":
        rec[1, 13] = rec[1, 12] + 64         # mm inside x1
    elif case == "cross_layer_overlap":
        rec[2, 14] = rec[0, 15]              # layer 2's xout on layer 0's o_next
    elif case == "misaligned":
        rec[0, 12] += 8
    elif case == "plan_misaligned":
        plan = 4104
    D, yld = 3072, 0
    if case.startswith("head"):
        D, yld = 1024, 8256
        rec[nl - 1, 7:10] = 256                          # the head's norm, weights, scales
        rec[nl - 1, 16] = (1 << 40)                      # y
        if case == "head_not_last":
            rec[0, 16] = (1 << 41)
        elif case == "head_3072_wide":
            D = 3072
        elif case == "head_with_cache":
            rec[nl - 1, 10] = 256
        elif case == "head_overlaps":
            rec[nl - 1, 16] = rec[1, 12]                 # y on a layer's x1
    rc = L.ecd_layer_stack_plan(rec.ctypes.data, nl, 8, D, 8192, 8, 4, 384, yld, plan, None)
    assert rc == _ffi.ECD_EINVAL


def test_python_wrappers_refuse_cpu_tensors():
    """The product path has no CPU fallback: CPU tensors raise instead of computing."""
    import torch
    from estudiocanciones_amd.kernels import int8_mm, rms
    x = torch.zeros(2, 64, dtype=torch.float16)
    w = torch.zeros(8, 64, dtype=torch.int8)
    s = torch.ones(8, dtype=torch.float16)
    with pytest.raises(RuntimeError):
        int8_mm(x, w, s)
    with pytest.raises(RuntimeError):
        rms(x, torch.ones(64, dtype=torch.float16))


def test_gemm_rejects_x_beyond_32bit_offsets():
    """The prompt GEMM's per-lane load offsets are 32-bit: an x buffer of 2 GiB or more is
    refused with ECD_ENOTSUP before any launch."""
    from estudiocanciones_amd import _ffi
    L = _ffi.lib()
    # M = 2^17 rows of ldx = 2^13 halfs -> 2 GiB
    assert L.ecd_gemm_i8p(16, 8192, 16, 16, None, 0, 16, 64, 1 << 17, 64, 8192, None) == _ffi.ECD_ENOTSUP
    assert L.ecd_gemm_i8p_silu(16, 8192, 16, 16, 16, 64, 1 << 17, 32, 8192, None) == _ffi.ECD_ENOTSUP
    assert L.ecd_gemm_i8p_rope(16, 8192, 16, 16, 16, 16, 16, 16, 16, 1 << 17, 1, 8, 2, 64, 128,
                               8192, None) == _ffi.ECD_ENOTSUP


def test_layer_head_validates_before_launch():
    """The head launch (a stack's layer 0 rms + q|k|v + attention) rejects missing buffers, a
    misaligned sync region and more than 16 rows with ECD_EINVAL before any HIP call."""
    from estudiocanciones_amd import _ffi
    L = _ffi.lib()
    shape = (8, 3072, 8192, 1, 24, 8, 1024, 128, 1e-5, 0, None)
    assert L.ecd_layer_head(*([256] * 9), None, *([256] * 3), *shape) == _ffi.ECD_EINVAL  # no o_next
    assert L.ecd_layer_head(*([256] * 10), 16, 256, 256, *shape) == _ffi.ECD_EINVAL  # sync 16-aligned
    assert L.ecd_layer_head(*([256] * 12), None, *shape) == _ffi.ECD_EINVAL  # no workspace
    assert L.ecd_layer_head(*([256] * 13), 17, 3072, 8192, 1, 24, 8, 1024, 128, 1e-5, 0,
                            None) == _ffi.ECD_EINVAL  # M > 16


def test_gemm_rope_validates_before_launch():
    """The q|k|v GEMM with the RoPE epilogue rejects bad shapes on the host (ECD_EINVAL, nothing
    launched): head_dim not a multiple of 4, Hq not a multiple of Hk, K not a multiple of 64,
    a missing position vector, a misaligned rope table."""
    from estudiocanciones_amd import _ffi
    L = _ffi.lib()
    E = _ffi.ECD_EINVAL
    ok = dict(x=16, ldx=1024, wp=16, s=16, rope=16, pos=16, q=16, kc=16, vc=16, M=64, S=1, Hq=8,
              Hk=2, L=64, HD=128, K=1024)

    def call(**kw):
        a = dict(ok, **kw)
        return L.ecd_gemm_i8p_rope(a["x"], a["ldx"], a["wp"], a["s"], a["rope"], a["pos"], a["q"],
                                   a["kc"], a["vc"], a["M"], a["S"], a["Hq"], a["Hk"], a["L"],
                                   a["HD"], a["K"], None)
    assert call(HD=126) == E
    assert call(Hq=7) == E
    assert call(K=1000, ldx=1000) == E
    assert call(pos=None) == E
    assert call(rope=8) == E
    assert call(M=0) == E


def test_noalloc_attention_refuses_oversized_workspace():
    """The static-workspace attention returns ECD_ENOMEM on the host, before any HIP call, when
    its split partials exceed the 8 MiB array (64 rows x 32 heads x 32 splits x head_dim 512)."""
    from estudiocanciones_amd import _ffi
    L = _ffi.lib()
    assert L.ecd_decode_attn_noalloc(16, 16, 16, 16, 16, 64, 1, 32, 8, 8192, 512, 32, 0.1,
                                     None) == _ffi.ECD_ENOMEM
