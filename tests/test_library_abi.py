"""The C ABI: header declarations, exported symbols and host-side checks.

No kernel is launched here: only entry points that never touch the device
(version, launch-table queries, workspace sizing, argument validation that
fails before any launch) are called.
"""

from __future__ import annotations

import ctypes
import re
from pathlib import Path

import pytest

from solution.kernels.hip import _library

HEADER = Path(__file__).resolve().parents[1] / "include" / "shape_aware_hip.h"


def _declared_functions() -> set[str]:
    text = HEADER.read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return set(re.findall(r"\b(sah_[a-z_0-9]+)\s*\(", text))


def test_header_and_binding_agree():
    declared = _declared_functions()
    assert declared == set(_library.EXPORTED_SYMBOLS)


def test_library_exports_every_declared_symbol():
    if not _library.LIBRARY_PATH.exists():
        pytest.fail(f"{_library.LIBRARY_PATH} is not built; run __graft_entry__.build()")
    raw = ctypes.CDLL(str(_library.LIBRARY_PATH))
    for name in _declared_functions():
        assert hasattr(raw, name), name


def test_host_only_entry_points():
    library = _library.load_library()
    assert library.sah_abi_version() == _library.ABI_VERSION
    assert library.sah_causal_attention_launch_supported(128, 64, 4, 2) == 1
    assert library.sah_causal_attention_launch_supported(256, 64, 4, 1) == 1
    assert library.sah_causal_attention_launch_supported(64, 64, 4, 2) == 0
    assert library.sah_causal_attention_launch_supported(128, 64, 4, 3) == 1
    assert library.sah_causal_attention_launch_supported(256, 64, 4, 3) == 0
    assert library.sah_causal_attention_launch_supported(512, 64, 8, 2) == 1
    assert library.sah_causal_attention_launch_supported(512, 64, 4, 2) == 0
    assert library.sah_causal_attention_launch_supported(128, 64, 8, 3) == 0
    from solution.shape14.hip_streaming_dh64 import launch_config_is_valid

    for block_m in (64, 128, 256, 512, 1024):
        for block_n in (32, 64, 128):
            for warps in (2, 4, 8):
                for stages in (1, 2, 3, 4):
                    assert launch_config_is_valid(block_m, block_n, warps, stages) == bool(
                        library.sah_causal_attention_launch_supported(block_m, block_n, warps, stages)
                    ), (block_m, block_n, warps, stages)
    # Sequences of 16384 keys or more get a table of the largest key norm of
    # every 64-key tile (fp32, rounded up to 256 bytes) ...
    norms = -(-(2 * 16 * -(-100000 // 64) * 4) // 256) * 256
    assert norms == 200192
    # ... two tables of the largest |k| and |q| of every 512-row block
    # (fp32, together rounded up to 256 bytes) ...
    blocks = -(-(2 * 2 * 16 * -(-100000 // 512) * 4) // 256) * 256
    assert blocks == 50176
    # ... and every key times c in fp16, padded to 64 keys.  A head_dim-
    # contiguous V (the reference layout, e.g. the packed QKV view) is read
    # as given ...
    scaled_keys = 2 * 16 * 100032 * 64 * 2
    assert library.sah_causal_attention_workspace_bytes(2, 16, 100000, 64, 3072, 1, 2) == norms + blocks + scaled_keys
    # ... and a seq-contiguous V^T adds its key-major copy (S x 64 per head).
    assert library.sah_causal_attention_workspace_bytes(2, 16, 100000, 64, 1, 100032, 2) == (
        norms + blocks + scaled_keys + 2 * 16 * 100000 * 64 * 2
    )
    assert library.sah_causal_attention_workspace_bytes(1, 16, 16384, 64, 1, 16384, 1) == (
        16 * 256 * 4 + 2 * 16 * 32 * 4 + 16 * 16384 * 128 + 16 * 16384 * 128
    )
    # The tables and scaled keys start at 4096 keys.
    assert library.sah_causal_attention_workspace_bytes(1, 2, 4096, 64, 64, 1, 2) == 512 + 256 + 2 * 4096 * 128
    assert library.sah_causal_attention_workspace_bytes(1, 2, 4095, 64, 64, 1, 2) == 0
    assert library.sah_causal_attention_workspace_bytes(1, 2, 4095, 64, 1, 4096, 2) == 2 * 4095 * 128
    # Shorter sequences need nothing with V as given, the copy with V^T.
    assert library.sah_causal_attention_workspace_bytes(8, 16, 2048, 64, 64, 1, 2) == 0
    assert library.sah_causal_attention_workspace_bytes(8, 16, 2048, 64, 1, 2048, 2) == 8 * 16 * 2048 * 64 * 2
    # fp32 reads K and V as given: no table, no copy
    assert library.sah_causal_attention_workspace_bytes(2, 16, 100000, 64, 64, 1, 0) == 0


def test_invalid_arguments_fail_before_launch():
    library = _library.load_library()
    status = library.sah_causal_attention_bsd(
        None, None, None, None, 1, 1, 1, 64, *([0] * 12), 0.125, 2, 128, 64, 4, 2, None, 0, None
    )
    assert status == _library.SAH_ERR_INVALID_ARGUMENT
    assert b"non-null" in library.sah_last_error()
    fake = ctypes.c_void_p(4096)  # never dereferenced: validation fails first
    status = library.sah_causal_attention_bsd(
        fake, fake, fake, fake, 1, 1, 16, 32, *([0] * 12), 0.125, 2, 128, 64, 4, 2, None, 0, None
    )
    assert status == _library.SAH_ERR_UNSUPPORTED and b"head_dim" in library.sah_last_error()
    # Tiles of 64 key rows of K and of V are addressed at 32-bit offsets: key
    # and value row strides outside [0, 2^24) elements are refused before any
    # launch.
    def attend(seq, k_ss, v_ss, v_sd, workspace=None, workspace_bytes=0):
        return library.sah_causal_attention_bsd(
            fake, fake, fake, fake, 1, 1, seq, 64, 0, 0, 64, 0, 0, k_ss, 0, 0, v_ss, v_sd, 0, 64,
            0.125, 2, 128, 64, 4, 2, workspace, workspace_bytes, None)

    for k_ss, v_ss in ((-64, 64), (1 << 24, 64), (64, 1 << 24), (64, -64)):
        assert attend(1000, k_ss, v_ss, 1) == _library.SAH_ERR_UNSUPPORTED, (k_ss, v_ss)
        assert b"32-bit tile offsets" in library.sah_last_error()
    # The preparation and V-copy launches put batch * heads on the grid's y
    # axis: more than 65535 is refused before any launch.
    for seq, v_ss, v_sd in ((100, 1, 104), (5000, 64, 1)):
        need = library.sah_causal_attention_workspace_bytes(65536, 1, seq, 64, v_ss, v_sd, 2)
        assert need > 0
        status = library.sah_causal_attention_bsd(
            fake, fake, fake, fake, 65536, 1, seq, 64, 0, 0, 64, 0, 0, 64, 0, 0, v_ss, v_sd, 0, 64,
            0.125, 2, 128, 64, 4, 2, fake, need, None)
        assert status == _library.SAH_ERR_UNSUPPORTED, (seq, status)
        assert b"65535 batch*heads" in library.sah_last_error()
    status = library.sah_residual_norm(
        fake, fake, None, None, fake, fake, 4, 1000, 1e-5, 2, 2, 2, 0, 0, 4, 4, None
    )
    assert status == _library.SAH_ERR_UNSUPPORTED
    status = library.sah_norm(fake, None, None, fake, 4, 1024, 1e-5, 2, 2, 0, 7, 4, 4, None)
    assert status == _library.SAH_ERR_INVALID_ARGUMENT and b"norm kind" in library.sah_last_error()
    status = library.sah_norm(fake, None, None, fake, 4, 1024, 1e-5, 2, 2, 0, 0, 3, 2, None)
    assert status == _library.SAH_ERR_UNSUPPORTED
    with pytest.raises(_library.HipLibraryError, match="status 2"):
        _library.check_status(_library.SAH_ERR_UNSUPPORTED, "probe")


def test_custom_op_has_a_fake_implementation():
    """The attention op traces on meta tensors (no kernel runs)."""

    import torch

    from solution.shape14 import hip_streaming_dh64  # noqa: F401 - registers the op

    q = torch.empty(2, 16, 1000, 64, device="meta", dtype=torch.bfloat16)
    out = torch.ops.shape_aware_hip.streaming_dh64_causal_attention_bsd(q, q, q, 0.125, 128, 64, 4, 2)
    assert out.shape == (2, 1000, 1024) and out.device.type == "meta"


def test_linear_entry_validates_before_launch():
    """sah_linear's launch table and argument checks (no kernel runs)."""

    from solution.kernels.ffn.hip_linear_gelu import launch_config_is_valid

    library = _library.load_library()
    assert library.sah_linear_launch_supported(256, 256, 64, 8, 2) == 1
    for launch in [(128, 128, 64, 8, 2), (256, 256, 32, 8, 2), (256, 256, 64, 4, 2), (256, 256, 64, 8, 3)]:
        assert library.sah_linear_launch_supported(*launch) == 0
        assert not launch_config_is_valid(*launch)
    assert launch_config_is_valid(256, 256, 64, 8, 2)
    assert not launch_config_is_valid(True, 256, 64, 8, 2)
    fake = ctypes.c_void_p(4096)  # never dereferenced: validation fails first
    args = dict(rows=4, k=1024, n=4096, ldx=1024, ldy=4096, dtype=2, act=1)

    def call(**over):
        a = {**args, **over}
        launch = over.get("launch", (256, 256, 64, 8, 2))
        return library.sah_linear(fake, fake, None, fake, a["rows"], a["k"], a["n"], a["ldx"], a["ldy"],
                                  a["dtype"], a["act"], *launch, None)

    assert call(launch=(128, 128, 64, 8, 2)) == _library.SAH_ERR_UNSUPPORTED
    assert call(k=1000) == _library.SAH_ERR_UNSUPPORTED and b"multiple" in library.sah_last_error()
    assert call(n=1000) == _library.SAH_ERR_UNSUPPORTED
    assert call(dtype=0) == _library.SAH_ERR_UNSUPPORTED
    assert call(act=5) == _library.SAH_ERR_INVALID_ARGUMENT
    assert call(ldx=1020) == _library.SAH_ERR_INVALID_ARGUMENT
    assert call(rows=-1) == _library.SAH_ERR_INVALID_ARGUMENT
    assert call(rows=0) == _library.SAH_OK  # nothing to do, nothing launched
    misaligned = ctypes.c_void_p(4096 + 8)
    status = library.sah_linear(misaligned, fake, None, fake, 4, 1024, 4096, 1024, 4096, 2, 1, 256, 256, 64, 8, 2, None)
    assert status == _library.SAH_ERR_INVALID_ARGUMENT and b"aligned" in library.sah_last_error()


def test_gelu_entry_validates_before_launch():
    from solution.kernels.ffn.hip_exact_gelu import launch_config_is_valid

    library = _library.load_library()
    for block_size in (256, 512, 1024, 2048, 4096, 8192, 16384, 3000):
        for warps in (1, 2, 3, 4, 8):
            assert launch_config_is_valid(block_size, warps) == bool(
                library.sah_gelu_launch_supported(block_size, warps)
            ), (block_size, warps)
    fake = ctypes.c_void_p(4096)  # never dereferenced: validation fails first
    assert library.sah_gelu(fake, fake, 10, 2, 256, 4, None) == _library.SAH_ERR_UNSUPPORTED
    assert library.sah_gelu(fake, fake, 10, 0, 4096, 4, None) == _library.SAH_ERR_UNSUPPORTED
    assert library.sah_gelu(fake, fake, -1, 2, 4096, 4, None) == _library.SAH_ERR_INVALID_ARGUMENT
    assert library.sah_gelu(fake, fake, 0, 2, 4096, 4, None) == _library.SAH_OK
    status = library.sah_gelu(ctypes.c_void_p(4096 + 2), fake, 10, 2, 4096, 4, None)
    assert status == _library.SAH_ERR_INVALID_ARGUMENT and b"aligned" in library.sah_last_error()


def test_qkv_projection_entry_validates_before_launch():
    """sah_qkv_projection's launch table and argument checks (no kernel runs)."""

    from solution.kernels.projection.hip_qkv_layout import launch_config_is_valid, supported_shape

    library = _library.load_library()
    assert library.sah_qkv_launch_supported(256, 256, 64, 8) == 1
    assert launch_config_is_valid(256, 256, 64, 8)
    for launch in [(64, 32, 32, 4), (128, 256, 64, 8), (256, 256, 32, 8), (256, 256, 64, 4)]:
        assert library.sah_qkv_launch_supported(*launch) == 0
        assert not launch_config_is_valid(*launch)
    assert not launch_config_is_valid(256, 256, 64, True)
    # d_model a multiple of 256, head_dim a multiple of 8
    assert supported_shape(1024, 16) and supported_shape(512, 8) and supported_shape(2048, 32)
    assert not supported_shape(32, 4) and not supported_shape(640, 10) and not supported_shape(1024, 256)
    fake = ctypes.c_void_p(4096)  # never dereferenced: validation fails first
    base = dict(batch=2, seq=100, d=1024, heads=16, ldx=1024, layout=_library.SAH_QKV_VALUE_SEQ_MAJOR,
                ldv=104, dtype=2, launch=(256, 256, 64, 8))

    def call(x=fake, **over):
        a = {**base, **over}
        return library.sah_qkv_projection(x, fake, None, fake, fake, fake, a["batch"], a["seq"], a["d"],
                                          a["heads"], a["ldx"], a["layout"], a["ldv"], a["dtype"],
                                          *a["launch"], None)

    assert call(launch=(64, 32, 32, 4)) == _library.SAH_ERR_UNSUPPORTED
    assert call(dtype=0) == _library.SAH_ERR_UNSUPPORTED
    assert call(d=640, heads=10, ldx=640) == _library.SAH_ERR_UNSUPPORTED and b"multiple" in library.sah_last_error()
    assert call(heads=256) == _library.SAH_ERR_UNSUPPORTED  # head_dim 4
    assert call(layout=7) == _library.SAH_ERR_INVALID_ARGUMENT
    assert call(ldv=96) == _library.SAH_ERR_INVALID_ARGUMENT  # below seq_len
    assert call(ldv=101) == _library.SAH_ERR_INVALID_ARGUMENT  # not a multiple of 8
    assert call(ldx=1000) == _library.SAH_ERR_INVALID_ARGUMENT
    assert call(batch=-1) == _library.SAH_ERR_INVALID_ARGUMENT
    assert call(seq=0) == _library.SAH_ERR_INVALID_ARGUMENT
    assert call(batch=40000, seq=100000, ldv=100000) == _library.SAH_ERR_UNSUPPORTED  # 4e9 tokens
    assert call(batch=0) == _library.SAH_OK  # nothing to do, nothing launched
    assert call(layout=_library.SAH_QKV_VALUE_BHSD, ldv=0, batch=0) == _library.SAH_OK
    status = call(x=ctypes.c_void_p(4096 + 8))
    assert status == _library.SAH_ERR_INVALID_ARGUMENT and b"aligned" in library.sah_last_error()


def test_norm_qkv_projection_entry_validates_before_launch():
    """sah_norm_qkv_projection: the projection's checks (reported under its
    own name) plus the LayerNorm's, all before any kernel runs."""

    library = _library.load_library()
    fake = ctypes.c_void_p(4096)  # never dereferenced: validation fails first
    base = dict(batch=2, seq=100, d=1024, heads=16, ldx=1024, layout=_library.SAH_QKV_VALUE_SEQ_MAJOR,
                ldv=104, dtype=2, launch=(256, 256, 64, 8), ln_w=fake, ln_b=fake, eps=1e-5, ws=fake, ws_bytes=1600)

    def call(**over):
        a = {**base, **over}
        return library.sah_norm_qkv_projection(fake, a["ln_w"], a["ln_b"], a["eps"], fake, None, fake, fake, fake,
                                               a["batch"], a["seq"], a["d"], a["heads"], a["ldx"], a["layout"],
                                               a["ldv"], a["dtype"], *a["launch"], a["ws"], a["ws_bytes"], None)

    assert call(ln_b=None) == _library.SAH_ERR_INVALID_ARGUMENT and b"both required" in library.sah_last_error()
    assert call(ln_w=None, ln_b=None) == _library.SAH_ERR_INVALID_ARGUMENT
    assert call(ln_w=ctypes.c_void_p(4096 + 8)) == _library.SAH_ERR_INVALID_ARGUMENT
    assert call(eps=float("nan")) == _library.SAH_ERR_INVALID_ARGUMENT
    assert call(eps=-1e-5) == _library.SAH_ERR_INVALID_ARGUMENT
    # widths with statistics instantiated: 512, 1024, 2048, 4096
    assert call(d=768, heads=12, ldx=768) == _library.SAH_ERR_UNSUPPORTED
    assert b"512, 1024, 2048 or 4096" in library.sah_last_error()
    assert call(d=8192, heads=128, ldx=8192) == _library.SAH_ERR_UNSUPPORTED
    # the projection's own checks, named for this entry point
    assert call(launch=(64, 32, 32, 4)) == _library.SAH_ERR_UNSUPPORTED
    assert library.sah_last_error().startswith(b"sah_norm_qkv_projection:")
    assert call(ldx=1000) == _library.SAH_ERR_INVALID_ARGUMENT
    assert call(batch=0) == _library.SAH_OK
    assert call(batch=0, ln_b=None) == _library.SAH_ERR_INVALID_ARGUMENT  # checked even with nothing to do
    # the statistics workspace: 8 bytes per token, 16-byte aligned
    assert library.sah_norm_qkv_workspace_bytes(2, 100) == 1600
    assert library.sah_norm_qkv_workspace_bytes(0, 100) == 0 and library.sah_norm_qkv_workspace_bytes(2, -1) == 0
    assert library.sah_norm_qkv_workspace_bytes(2**40, 2**30) == 0  # no overflow
    assert call(ws_bytes=1599) == _library.SAH_ERR_WORKSPACE and b"1600" in library.sah_last_error()
    assert call(ws=None) == _library.SAH_ERR_WORKSPACE
    assert call(ws=ctypes.c_void_p(4096 + 8)) == _library.SAH_ERR_WORKSPACE


def test_mlp_residual_norm_entry_validates_before_launch():
    """sah_mlp_residual_norm's launch table and argument checks (no kernel runs)."""

    from solution.kernels.boundary.hip_mlp_residual_norm import launch_config_is_valid, supported_shape

    library = _library.load_library()
    for width in (128, 256):
        assert library.sah_mlp_residual_norm_launch_supported(width, 64, 4) == 1
        assert launch_config_is_valid(width, 64, 4)
    for launch in [(512, 64, 4), (256, 32, 4), (256, 64, 8), (1024, 64, 4)]:
        assert library.sah_mlp_residual_norm_launch_supported(*launch) == 0
        assert not launch_config_is_valid(*launch)
    assert supported_shape(128, 128) and supported_shape(256, 1024) and not supported_shape(256, 1000)
    assert not supported_shape(512, 2048)
    fake = ctypes.c_void_p(4096)  # never dereferenced: validation fails first
    base = dict(rows=100, width=256, ffn=1024, ldx=256, eps=1e-5, dtype=2, kind=_library.SAH_NORM_LAYER,
                launch=(64, 4), x=fake, b1=None)

    def call(**over):
        a = {**base, **over}
        return library.sah_mlp_residual_norm(a["x"], fake, a["b1"], fake, None, fake, None, None, fake, fake,
                                             a["rows"], a["width"], a["ffn"], a["ldx"], a["eps"], a["dtype"],
                                             a["kind"], *a["launch"], None)

    assert call(width=512, ldx=512) == _library.SAH_ERR_UNSUPPORTED
    assert library.sah_last_error().startswith(b"sah_mlp_residual_norm:")
    assert call(launch=(32, 4)) == _library.SAH_ERR_UNSUPPORTED
    assert call(dtype=0) == _library.SAH_ERR_UNSUPPORTED
    assert call(kind=7) == _library.SAH_ERR_INVALID_ARGUMENT
    assert call(ffn=1000) == _library.SAH_ERR_INVALID_ARGUMENT
    assert call(ffn=0) == _library.SAH_ERR_INVALID_ARGUMENT
    assert call(rows=-1) == _library.SAH_ERR_INVALID_ARGUMENT
    assert call(ldx=200) == _library.SAH_ERR_INVALID_ARGUMENT
    assert call(eps=float("inf")) == _library.SAH_ERR_INVALID_ARGUMENT
    assert call(rows=0) == _library.SAH_OK  # nothing to do, nothing launched
    assert call(x=None) == _library.SAH_ERR_INVALID_ARGUMENT
    assert call(x=ctypes.c_void_p(4096 + 8)) == _library.SAH_ERR_INVALID_ARGUMENT
    assert call(b1=ctypes.c_void_p(4096 + 4)) == _library.SAH_ERR_INVALID_ARGUMENT
