"""The C ABI library (no GPU needed): it loads, exports every entry point include/sa.h declares, and
its host-side sizing/validation entry points behave; the Python API's input checks run on the CPU."""

from __future__ import annotations

import ctypes
import os
import re

import pytest
import torch

from selective_attention import _lib, kernels

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "sa.h")


def _declared():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(sa_[a-z_0-9]+)\s*\(", text)))


def test_header_declares_the_bound_functions():
    assert _declared() == sorted(_lib.SIGNATURES)


def test_library_loads_and_exports_every_declared_symbol():
    lib = _lib.load()
    for name in _declared():
        assert hasattr(lib, name), name
    assert lib.sa_abi_version() >= 1


def test_status_strings():
    lib = _lib.load()
    for code in (0, -1, -2, -3, -4, -5, -6):
        assert lib.sa_status_string(code)
    assert b"head_dim" in lib.sa_status_string(-2)


def test_workspace_sizes():
    lib = _lib.load()
    assert lib.sa_transposed_ld(1) == 64 and lib.sa_transposed_ld(64) == 64 and lib.sa_transposed_ld(65) == 128
    # the forward's scratch is V^T, except where the head-dim-64 bf16 kernel (one or two heads per
    # wavefront, the default) reads the V rows themselves
    assert lib.sa_forward_workspace_bytes(1, 16, 16384, 64, 0, 0) == 0
    assert lib.sa_forward_workspace_bytes(1, 15, 16384, 64, 0, 0) == 0
    fw = lib.sa_forward_workspace_bytes(1, 16, 16384, 64, 0, 4)
    assert fw >= 16 * 64 * 16384 * 2 and fw % 256 == 0
    assert lib.sa_forward_workspace_bytes(1, 16, 16384, 32, 0, 0) >= 16 * 32 * 16384 * 2
    assert lib.sa_forward_workspace_bytes(1, 16, 16384, 64, 1, 0) >= 16 * 64 * 16384 * 4
    bw = lib.sa_backward_workspace_bytes(1, 16, 16384, 64, 0, 0)
    # the 16 head groups' U checkpoints (the causal part of each 512 x 16384 plane: 32 x 512 x 513 / 2
    # floats), head 0's fp32 dq and dk and the other 15 groups' shares of them (one slot each, so the
    # finishing sum runs in a fixed order), lse and -dbar; no transposed copies (at bf16 head dim 64
    # the kernels read Q, dO and K transposed from LDS)
    tri = 16 * 512 * 513
    fixed = 16 * tri * 4 + (2 + 2 * 15) * 16384 * 64 * 4 + 2 * 16 * 16384 * 4
    assert bw >= fixed and bw % 256 == 0
    assert bw < fixed + 4096
    # other head dims (and fp32 storage) keep the Q^T, dO^T and K^T copies
    bw32 = lib.sa_backward_workspace_bytes(1, 16, 16384, 32, 0, 1)
    assert bw32 >= 3 * 16 * 32 * 16384 * 2 + 16 * tri * 4
    bwf = lib.sa_backward_workspace_bytes(1, 16, 16384, 64, 1, 0)
    assert bwf >= 3 * 16 * 64 * 16384 * 4 + fixed
    dw = lib.sa_decode_workspace_bytes(1, 16, 131072, 64)
    assert dw >= 16 * (131072 // 64) * 66 * 4 and dw % 256 == 0   # one (m, l, o[64]) per 64 keys and head
    assert lib.sa_decode_workspace_bytes(0, 16, 100, 64) < 0


def test_decode_rejects_invalid_arguments():
    lib = _lib.load()
    fake = 1 << 20   # never dereferenced: validation fails first
    args = [fake] * 5 + [128, fake, 1 << 30, 1, 4, 1, 100, 0, 64, 0.125, 0, 1, None]
    bad = list(args)
    bad[10] = 3          # groups does not divide heads
    assert lib.sa_decode(*bad) == -1
    bad = list(args)
    bad[5] = 99          # state row shorter than t
    assert lib.sa_decode(*bad) == -1
    bad = list(args)
    bad[13] = 48         # head_dim
    assert lib.sa_decode(*bad) == -2
    bad = list(args)
    bad[15] = 9          # dtype
    assert lib.sa_decode(*bad) == -3
    bad = list(args)
    bad[7] = 8           # workspace too small
    assert lib.sa_decode(*bad) == -4
    bad = list(args)
    bad[16] = 0          # exempt
    assert lib.sa_decode(*bad) == -1


def test_decode_noalloc_rejects_before_touching_a_device():
    """The allocation-free decode checks its arguments as sa_decode does, and refuses a step whose
    scratch exceeds its fixed array, before any device call."""
    lib = _lib.load()
    fake = 1 << 20
    args = [fake] * 5 + [128, 1, 4, 1, 100, 0, 64, 0.125, 0, 1, None]
    bad = list(args)
    bad[8] = 3           # groups does not divide heads
    assert lib.sa_decode_noalloc(*bad) == -1
    bad = list(args)
    bad[11] = 48         # head_dim
    assert lib.sa_decode_noalloc(*bad) == -2
    bad = list(args)
    bad[13] = 9          # dtype
    assert lib.sa_decode_noalloc(*bad) == -3
    t = 1 << 21          # 2M keys at 16 heads: about 160 MiB of scratch
    assert lib.sa_decode_workspace_bytes(1, 16, t, 64) > _lib.DECODE_SCRATCH_BYTES
    big = [fake] * 5 + [t, 1, 16, 1, t, 0, 64, 0.125, 0, 1, None]
    assert lib.sa_decode_noalloc(*big) == -6
    assert b"scratch" in lib.sa_status_string(-6)


def test_invalid_arguments_are_rejected_before_any_launch():
    """Host validation in C: no pointer is dereferenced, no kernel launched."""
    lib = _lib.load()
    fake = 1 << 20   # never dereferenced: validation fails first
    args = [fake] * 9 + [16, fake, 1 << 30, 1, 4, 16, 16, 0, 0, 64, 0.125, 0, 1, 0, 0, 0, None]
    bad = list(args)
    bad[16] = 5          # q_offset + tq != tk
    assert lib.sa_forward(*bad) == -1
    bad = list(args)
    bad[18] = 48         # head_dim
    assert lib.sa_forward(*bad) == -2
    bad = list(args)
    bad[17] = 16 * 64 - 8   # kv_stride below tk * head_dim
    assert lib.sa_forward(*bad) == -1
    bad = list(args)
    bad[20] = 7          # dtype
    assert lib.sa_forward(*bad) == -3
    bad = list(args)
    bad[11] = 16         # workspace too small (four heads per wavefront: fwd_kernel reads V^T)
    bad[22] = 4
    assert lib.sa_forward(*bad) == -4
    bad = list(args)
    bad[21] = 0          # exempt
    assert lib.sa_forward(*bad) == -1
    bargs = [fake] * 12 + [1 << 30, 1, 4, 16, 64, 0.125, 0, 1, 1, 0, None]
    bad = list(bargs)
    bad[16] = 100
    assert lib.sa_backward(*bad) == -2
    bad = list(bargs)
    bad[17] = -1.0
    assert lib.sa_backward(*bad) == -1
    bad = list(bargs)
    bad[19] = 5          # grad dtype
    assert lib.sa_backward(*bad) == -3


def test_strided_views_are_validated_before_any_launch():
    """sa_forward_strided / sa_backward_strided check every view (no pointer dereferenced)."""
    lib = _lib.load()
    fake = 1 << 20
    V = _lib.ViewStrides
    good = V(16 * 3 * 4 * 64, 64, 3 * 4 * 64)   # a packed (B, T=16, 3, H=4, 64) projection
    ws = 1 << 30

    def fwd(qs=good, ks=good, vs=good, y=None, ys=None, q=fake):
        return lib.sa_forward_strided(q, qs, fake + 512, ks, fake + 1024, vs, fake, y, ys, fake, fake, fake, None,
                                      fake, 16, fake, ws, 1, 4, 16, 16, 0, 64, 0.125, 0, 1, 0, 0, 0, None)

    assert fwd(qs=V(0, 64, 32)) == -1                     # row stride below head_dim
    assert fwd(ks=V(16 * 768, 64, 770)) == -1             # row stride not a multiple of 8 elements
    assert fwd(q=fake + 8) == -1                          # pointer not 16-byte aligned
    assert fwd(y=fake, ys=V(16 * 256, 32, 256)) == -1     # output heads overlap
    assert fwd(y=fake, ys=None) == -1                     # output without a view
    assert fwd(qs=V(16 * 768, 64, 1 << 27)) == -1         # rows past the 2 GiB a head may span

    def bwd(dqs=good, dos=good, dq=fake, dv=fake):
        return lib.sa_backward_strided(fake, good, fake, good, fake, good, fake, fake, dos, fake, fake, fake,
                                       dq, dqs, fake, good, dv, good, fake, ws, 1, 4, 16, 64, 0.125, 0, 0, 1,
                                       0, None)

    assert bwd(dqs=V(0, 16, 768)) == -1                   # gradient heads overlap
    assert bwd(dos=V(0, 64, 60)) == -1                    # dout row stride below head_dim
    # gradients are written in 8- and 16-byte pieces straight into the views
    assert bwd(dq=fake + 8) == -1                         # gradient pointer not 16-byte aligned
    assert bwd(dv=fake + 2) == -1


def test_api_checks_on_cpu_tensors():
    q = torch.randn(1, 2, 16, 32)
    assert not kernels.supported(q)
    with pytest.raises(ValueError, match="CUDA"):
        kernels.check_inputs(q, q, q)
    with pytest.raises(ValueError, match="must all be"):
        kernels.check_inputs(q, q[:, :, :8], q)
    with pytest.raises(ValueError, match="dot_precision"):
        kernels._resolve_precision("fp8", torch.float32)
    assert kernels._resolve_precision(None, torch.bfloat16) == _lib.DTYPE_BF16
    assert kernels._resolve_precision(None, torch.float16) == _lib.DTYPE_F32
    with pytest.raises(ValueError, match="exempt"):
        kernels._check_exempt(0)
    with pytest.raises(ValueError, match="bwd_group"):
        kernels._check_bwd_group(3)
    with pytest.raises(ValueError, match="damp"):
        kernels._damp_mode("cubic", 10)
    with pytest.raises(ValueError, match="train_len"):
        kernels._damp_mode("linear", 0)
    with pytest.raises(ValueError, match="multiples"):
        kernels._check_blocks(48, 32)


def test_custom_ops_have_fake_shape_functions():
    """The C-ABI calls are torch.library custom ops whose fake (meta) kernels give the shapes and
    dtypes torch.compile traces with; no GPU is needed to run them."""
    from torch._subclasses.fake_tensor import FakeTensorMode

    ops = torch.ops.selective_attention
    with FakeTensorMode():
        q = torch.empty(2, 4, 100, 32, dtype=torch.bfloat16, device="meta")
        out, rmax, rden, carry, total = ops.forward(q, q, q, 0.125, 1, 0, 0, 0)
        assert out.shape == (2, 4, 100, 32) and out.dtype == torch.float32
        assert rmax.shape == rden.shape == (2, 4, 100) and carry.shape == (2, 4, 100) and total.shape == (2, 100)
        for flag, dt in ((True, torch.bfloat16), (False, torch.float32)):
            grads = ops.backward(q, q, q, out, q, rmax, rden, carry, 0.125, 1, 0, flag)
            assert all(g.shape == q.shape and g.dtype == dt for g in grads)
        qkv = torch.empty(2, 70, 3 * 4 * 64, dtype=torch.bfloat16, device="meta")
        y, o, m, d, c = ops.qkv_forward(qkv, 4, 1)
        assert y.shape == (2, 70, 256) and y.dtype == torch.bfloat16 and o.shape == (2, 4, 70, 64)
        assert c.shape == (2, 3, 70)
        assert ops.qkv_backward(qkv, y, o, m, d, c, 4, 1).shape == qkv.shape


def test_packed_form_stays_within_32_bit_row_offsets():
    """One head's rows of the packed projection are addressed with 32-bit byte offsets at the packed
    row stride 3 * H * D: past 2 GiB the fused form is refused, so the slot takes the split-heads
    path (rows D apart), which runs ~3 H times longer sequences."""
    c3 = 3 * 1024   # d1024 / 16 heads
    assert kernels._packed_rows_fit(300_000, c3, 2)
    assert not kernels._packed_rows_fit(350_000, c3, 2)   # (T + 64) * 3072 * 2 bytes >= 2^31
    assert not kernels._packed_rows_fit(175_000, c3, 4)
