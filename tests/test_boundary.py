"""The C ABI boundary, checked without a GPU: the library loads, exports
every symbol the headers under include/ declare, and turns bad arguments into status
codes (never a crash) before it touches a device."""

import ctypes
import re
from pathlib import Path

import numpy as np
import pytest
import torch

ROOT = Path(__file__).resolve().parents[1]
HEADERS = sorted((ROOT / "include").glob("*.h"))

NO_GPU = not torch.cuda.is_available()


def declared_functions(headers=None):
    names = set()
    for h in headers or HEADERS:
        text = re.sub(r"/\*.*?\*/", "", h.read_text(), flags=re.S)
        names.update(re.findall(r"\b(fmoe_[a-z0-9_]+)\s*\(", text))
    return sorted(names)


def test_path_override_is_outside_the_product_header():
    product = declared_functions([ROOT / "include" / "fmoe.h"])
    assert not [n for n in product if "gemm_path" in n]
    assert "fmoe_set_gemm_path" in declared_functions([ROOT / "include" / "fmoe_diag.h"])


def test_header_declares_the_drop_in_entry_points():
    names = declared_functions()
    for required in ("fmoe_moe_ffn_block", "fmoe_mul_mat_id", "fmoe_swiglu", "fmoe_router",
                     "fmoe_permute", "fmoe_pack_expert_weights"):
        assert required in names


def test_library_exports_every_declared_symbol(fm):
    lib = fm.lowlevel.lib()
    missing = [n for n in declared_functions() if not hasattr(lib, n)]
    assert not missing, missing
    # and the Python binding types every one of them
    assert set(declared_functions()) == set(fm.lowlevel.SIGNATURES)


def test_abi_version(fm):
    text = (Path(__file__).resolve().parents[1] / "include" / "fmoe.h").read_text()
    declared = int(re.search(r"#define FMOE_ABI_VERSION (\d+)", text).group(1))
    assert declared == 3
    assert fm.lowlevel.lib().fmoe_abi_version() == declared


def test_single_hip_runtime(fm):
    # libfmoe binds to the runtime torch loaded (one libamdhip64 mapping)
    assert len(fm.hip_runtimes_loaded()) == 1, fm.hip_runtimes_loaded()


def st(fm, name, *args):
    return getattr(fm.lowlevel.lib(), name)(*args)


def test_argument_errors_before_device(fm):
    ll = fm.lowlevel
    # bad dtype
    assert st(fm, "fmoe_swiglu", None, None, None, 4, 9, None) == ll.ERR_DTYPE
    # bad shapes: n_expert 0, k > E, too many experts
    assert st(fm, "fmoe_router", None, None, 4, 8, 0, 1, 0, ll.F32, None, None, None) == ll.ERR_SHAPE
    assert st(fm, "fmoe_router", None, None, 4, 8, 4, 5, 0, ll.F32, None, None, None) == ll.ERR_SHAPE
    assert st(fm, "fmoe_router", None, None, 4, 8, 300, 2, 0, ll.F32, None, None, None) == ll.ERR_SHAPE
    assert "n_expert" in ll.last_error()
    # bad flag
    assert st(fm, "fmoe_router", None, None, 4, 8, 4, 2, 2, ll.F32, None, None, None) == ll.ERR_INVALID_ARGUMENT
    # null pointers with valid shapes
    assert st(fm, "fmoe_router", None, None, 4, 8, 4, 2, 0, ll.F32, None, None, None) == ll.ERR_INVALID_ARGUMENT
    # fp8 activations are not a thing
    assert st(fm, "fmoe_moe_ffn_block", None, None, None, None, None, None, None, None, ll.F8E4M3FN,
              None, 4, 4, 2, 8, 16, 0, ll.F8E4M3FN, None, 0, None) == ll.ERR_DTYPE
    # f32 activations with bf16 weights
    assert st(fm, "fmoe_moe_ffn_block", None, None, None, None, None, None, None, None, ll.BF16,
              None, 4, 4, 2, 8, 16, 0, ll.F32, None, 0, None) == ll.ERR_DTYPE
    # packing fp8 into bf16
    assert st(fm, "fmoe_pack_expert_weights", None, ll.F8E4M3FN, None, 4, 4, 2, ll.BF16, None, None,
              None) == ll.ERR_DTYPE
    # unknown GEMM path
    assert st(fm, "fmoe_set_gemm_path", 17) == ll.ERR_INVALID_ARGUMENT
    assert st(fm, "fmoe_get_gemm_path") == ll.PATH_AUTO


def test_workspace_too_small_is_reported(fm):
    ll = fm.lowlevel
    need = ll.lib().fmoe_moe_ffn_block_workspace_bytes(16, 8, 2, 64, 128, ll.BF16, ll.BF16)
    fake = ctypes.c_void_p(0x1000)  # never dereferenced: validation fails first
    r = st(fm, "fmoe_moe_ffn_block", fake, fake, fake, fake, fake, None, None, None, ll.BF16, fake,
           16, 8, 2, 64, 128, 0, ll.BF16, fake, need - 1, None)
    assert r == ll.ERR_WORKSPACE


def test_empty_batch_is_a_no_op(fm):
    ll = fm.lowlevel
    # n_tokens = 0 returns OK without touching pointers or the device
    assert st(fm, "fmoe_moe_ffn_block", None, None, None, None, None, None, None, None, ll.F32,
              None, 0, 4, 2, 8, 16, 0, ll.F32, None, 0, None) == ll.OK
    assert st(fm, "fmoe_router", None, None, 0, 8, 4, 2, 0, ll.F32, None, None, None) == ll.OK


def test_workspace_sizes(fm):
    lib = fm.lowlevel.lib()
    ll = fm.lowlevel
    a = lib.fmoe_moe_ffn_block_workspace_bytes(16, 8, 2, 4096, 14336, ll.BF16, ll.BF16)
    b = lib.fmoe_moe_ffn_block_workspace_bytes(4096, 8, 2, 4096, 14336, ll.BF16, ll.BF16)
    assert 0 < a < b
    assert b % 256 == 0
    assert lib.fmoe_moe_ffn_block_workspace_bytes(16, 8, 2, 4096, 14336, 9, ll.BF16) == 0
    # weights + a 256-row tail the tiled kernels may read past the last expert
    assert lib.fmoe_packed_weight_bytes(14336, 4096, 8, ll.BF16) == 14336 * 4096 * 8 * 2 + 256 * 4096 * 2
    assert lib.fmoe_packed_weight_bytes(14336, 4096, 8, ll.F8E4M3FN) == 14336 * 4096 * 8 + 256 * 4096 * 2
    assert lib.fmoe_mul_mat_id_workspace_bytes(64, 32, 8, 2, 16, ll.F32) > 0
    # permutation: an error word; above 2048 assignments also a histogram per
    # chunk of 2048 (n_expert + 1 counts each)
    assert lib.fmoe_permute_workspace_bytes(2, 1024, 8) == 256
    assert lib.fmoe_permute_workspace_bytes(8, 8192, 128) == 256 + (32 * 129 * 4 + 255) // 256 * 256


@pytest.mark.skipif(not NO_GPU, reason="checks the no-device path")
def test_layer_glue_entry_points(fm):
    """fmoe_rms_norm and fmoe_moe_ffn_sublayer validate before touching a device."""
    ll = fm.lowlevel
    lib = ll.lib()
    assert st(fm, "fmoe_rms_norm", None, None, 1e-6, None, 4, 8, ll.F8E4M3FN, None) == ll.ERR_DTYPE
    assert st(fm, "fmoe_rms_norm", None, None, 1e-6, None, 4, 0, ll.F32, None) == ll.ERR_SHAPE
    assert st(fm, "fmoe_rms_norm", None, None, 1e-6, None, 4, 8, ll.F32, None) == ll.ERR_INVALID_ARGUMENT
    assert st(fm, "fmoe_rms_norm", None, None, 1e-6, None, 0, 8, ll.F32, None) == ll.OK  # no rows
    # the sub-layer workspace is the block's plus the normalised rows
    blk = lib.fmoe_moe_ffn_block_workspace_bytes(300, 8, 2, 4096, 14336, ll.BF16, ll.BF16)
    sub = lib.fmoe_moe_ffn_sublayer_workspace_bytes(300, 8, 2, 4096, 14336, ll.BF16, ll.BF16)
    assert sub == blk + (300 * 4096 * 2 + 255) // 256 * 256
    fake = ctypes.c_void_p(0x1000)  # never dereferenced: validation fails first
    args = [fake, fake, fake, fake, fake, None, None, None, ll.BF16, fake, 16, 8, 2, 64, 128, 0, ll.BF16]
    # null norm weight
    assert st(fm, "fmoe_moe_ffn_sublayer", fake, None, 1e-6, *args[1:], fake, sub, None) == ll.ERR_INVALID_ARGUMENT
    # workspace sized for the block only
    need = lib.fmoe_moe_ffn_sublayer_workspace_bytes(16, 8, 2, 64, 128, ll.BF16, ll.BF16)
    blk16 = lib.fmoe_moe_ffn_block_workspace_bytes(16, 8, 2, 64, 128, ll.BF16, ll.BF16)
    assert need > blk16
    assert st(fm, "fmoe_moe_ffn_sublayer", fake, fake, 1e-6, *args[1:], fake, blk16, None) == ll.ERR_WORKSPACE
    # the block's own checks apply (f32 activations with bf16 weights)
    bad = list(args)
    bad[16] = ll.F32
    assert st(fm, "fmoe_moe_ffn_sublayer", fake, fake, 1e-6, *bad[1:], fake, need, None) == ll.ERR_DTYPE
    # Python side: shapes are checked before any device work
    with pytest.raises(ValueError):
        fm.rms_norm(np.zeros((4, 8), np.float32), np.zeros(7, np.float32))
    wr = np.zeros((4, 8), np.float32)
    w3 = np.zeros((16, 8, 4), np.float32)
    wd = np.zeros((8, 16, 4), np.float32)
    with pytest.raises(ValueError):
        fm.moe_ffn_sublayer(np.zeros((3, 8), np.float32), np.zeros(9, np.float32), 1e-6, wr, w3, w3, wd,
                            4, 2, 8, 16, False)
    with pytest.raises(TypeError):
        fm.moe_ffn_sublayer(np.zeros((3, 8), np.float64), np.zeros(8, np.float32), 1e-6, wr, w3, w3, wd,
                            4, 2, 8, 16, False)


def test_no_device_is_an_error_not_a_crash(fm):
    ll = fm.lowlevel
    fake = ctypes.c_void_p(0x1000)  # validation passes; the device check must fail before any launch
    r = st(fm, "fmoe_router", fake, fake, 4, 8, 4, 2, 0, ll.F32, fake, fake, None)
    assert r == ll.ERR_NO_DEVICE
    d = ctypes.c_int(-1)
    assert st(fm, "fmoe_device_check", ctypes.byref(d), None, 0) == ll.ERR_NO_DEVICE


def test_python_api_errors_without_device(fm):
    x = np.zeros((4, 8), np.float32)
    w3 = np.zeros((16, 8, 4), np.float32)
    wd = np.zeros((8, 16, 4), np.float32)
    wr = np.zeros((4, 8), np.float32)
    with pytest.raises(TypeError):
        fm.moe_ffn_block(x.astype(np.float64), wr, w3, w3, wd, 4, 2, 8, 16, False)
    with pytest.raises(ValueError):
        fm.moe_ffn_block(x, wr, w3, w3, wd, 4, 2, 9, 16, False)  # n_embd mismatch
    with pytest.raises(ValueError):
        fm.moe_ffn_block(x, wr, w3, w3, wd, 4, 5, 8, 16, False)  # k > E
    with pytest.raises(IndexError):
        fm.mul_mat_id(np.zeros((4, 3, 8), np.float32), np.zeros((3, 1, 2), np.float32),
                      np.array([[0, 8]], np.int32))
    with pytest.raises(IndexError):
        fm.mul_mat_id(np.zeros((4, 3, 8), np.float32), np.zeros((3, 1, 2), np.float32),
                      np.array([[-1, 0]], np.int32))
    with pytest.raises(ValueError):
        fm.mul_mat_id(np.zeros((4, 3, 8), np.float32), np.zeros((3, 2, 2), np.float32),
                      np.array([[0, 1]], np.int32))
    with pytest.raises(TypeError):
        fm.mul_mat_id(np.zeros((4, 3, 8), np.float32), np.zeros((3, 1, 2), np.float32),
                      np.array([[0.0, 1.0]]))
    with pytest.raises(ValueError):
        fm.swiglu(np.zeros((2, 3), np.float32), np.zeros((3, 2), np.float32))


@pytest.mark.parametrize("shape,dt", [((32, 64, 3), "bf16"), ((32, 128, 2), "fp8"), ((24, 40, 5), "bf16"),
                                      ((16, 96, 2), "fp8")])
def test_packed_layout_is_a_bijection(shape, dt):
    from helpers import packed_index

    idx = packed_index(*shape, dt).reshape(-1)
    assert np.array_equal(np.sort(idx), np.arange(idx.size))


def _bare_block(fm, n_embd=8):
    """A MoEFFNBlock shell holding only what its host-side checks read (no
    packed weights, so no device is needed)."""
    blk = fm.MoEFFNBlock.__new__(fm.MoEFFNBlock)
    blk.act = fm.lowlevel.BF16
    blk.n_embd = n_embd
    blk._ws = None
    blk._last = None
    return blk


def test_block_out_argument_is_checked(fm):
    """out= reaches the C ABI as a raw pointer that the combine kernel writes
    T * n_embd elements through: shape, dtype, device and contiguity are
    checked first."""
    blk = _bare_block(fm)
    cpu = torch.device("cpu")
    good = torch.empty((3, 8), dtype=torch.bfloat16)
    assert blk._check_out(good, 3, cpu) is good
    assert blk._check_out(None, 3, cpu).shape == (3, 8)
    for bad in (torch.empty((2, 8), dtype=torch.bfloat16),          # too few rows
                torch.empty((3, 9), dtype=torch.bfloat16),          # wrong width
                torch.empty((3, 8), dtype=torch.float32),           # wrong dtype
                torch.empty((8, 3), dtype=torch.bfloat16).t(),      # not contiguous
                torch.empty((24,), dtype=torch.bfloat16)):          # flat
        with pytest.raises(ValueError):
            blk._check_out(bad, 3, cpu)
    with pytest.raises(ValueError):
        blk._check_out(good, 3, torch.device("meta"))               # another device


def test_block_routing_needs_the_last_calls_token_count(fm):
    blk = _bare_block(fm)
    with pytest.raises(RuntimeError):
        blk.routing()
    blk._ws = torch.zeros(4096, dtype=torch.uint8)
    blk._last = None  # a call that raised before completing its launches
    with pytest.raises(RuntimeError):
        blk.routing(16)
    blk._last = 16
    with pytest.raises(ValueError):
        blk.routing(17)


def test_noalloc_block_rejects_oversize_before_device(fm):
    """fmoe_moe_ffn_block_noalloc checks its fixed scratch size (and its
    arguments) before it touches a device."""
    ll = fm.lowlevel
    lib = ll.lib()
    fake = ctypes.c_void_p(0x1000)  # never dereferenced
    need = lib.fmoe_moe_ffn_block_workspace_bytes(4096, 8, 2, 4096, 14336, ll.BF16, ll.BF16)
    assert need > ll.NOALLOC_SCRATCH_BYTES
    r = st(fm, "fmoe_moe_ffn_block_noalloc", fake, fake, fake, fake, fake, None, None, None, ll.BF16, fake,
           4096, 8, 2, 4096, 14336, 0, ll.BF16, None)
    assert r == ll.ERR_WORKSPACE and "FMOE_NOALLOC_SCRATCH_BYTES" in ll.last_error()
    assert st(fm, "fmoe_moe_ffn_block_noalloc", None, None, None, None, None, None, None, None, ll.BF16, None,
              0, 8, 2, 64, 128, 0, ll.BF16, None) == ll.OK  # no tokens
    assert st(fm, "fmoe_moe_ffn_block_noalloc", fake, None, fake, fake, fake, None, None, None, ll.BF16, fake,
              16, 8, 2, 64, 128, 0, ll.BF16, None) == ll.ERR_INVALID_ARGUMENT  # null router


def test_two_term_fp8_activations_workspace(fm):
    """FMOE_F8E4M3FN_A8X2 takes the FMOE_F8E4M3FN_A8 workspace plus a second
    code plane for the token rows and for the SwiGLU rows (n * (H + F) bytes
    at least); decode-sized batches need none of it."""
    ll = fm.lowlevel
    lib = ll.lib()
    T, E, k, H, F = 4096, 8, 2, 4096, 14336
    one = lib.fmoe_moe_ffn_block_workspace_bytes(T, E, k, H, F, ll.BF16, ll.F8E4M3FN_A8)
    two = lib.fmoe_moe_ffn_block_workspace_bytes(T, E, k, H, F, ll.BF16, ll.F8E4M3FN_A8X2)
    assert two - one >= T * k * (H + F)
    dec = [lib.fmoe_moe_ffn_block_workspace_bytes(16, E, k, H, F, ll.BF16, d)
           for d in (ll.F8E4M3FN, ll.F8E4M3FN_A8, ll.F8E4M3FN_A8X2)]
    assert dec[0] == dec[1] == dec[2]
    assert lib.fmoe_moe_ffn_block_workspace_bytes(T, E, k, H, F, ll.BF16, 5) == 0
