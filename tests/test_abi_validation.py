"""Argument validation of the C ABI, on the CPU.

Every case here is rejected (or is an empty call) before the library touches the HIP runtime, so
the calls are safe without a GPU. Each must return the documented status: DX_ERR_INVALID for
malformed arguments, DX_ERR_UNSUPPORTED for shapes the kernels do not cover, and DX_OK for an
empty problem. dx_last_error must then name the entry point."""

from __future__ import annotations

import ctypes

import pytest

from deciax_amd import _lib

P = ctypes.c_void_p(0x10000)  # an aligned, non-null stand-in; never dereferenced by these calls
NUL = None


def lib():
    return _lib.lib()


def status(name: str, *args) -> int:
    return getattr(lib(), name)(*args)


def check(name: str, want: int, *args) -> None:
    got = status(name, *args)
    assert got == want, (name, got, want, lib().dx_last_error())
    if want != _lib.DX_OK:
        assert name.removeprefix("dx_").split("_f32")[0].split("_")[0] in lib().dx_last_error().decode()


def qkv(rows=8, hidden=512, hq=4, hkv=2, d=128, ldx=512, ld_qk=768, vt_ld=64, max_pos=64, first=P):
    return ("dx_qkv_rope", first, P, P, P, P, P, P, P, rows, hidden, hq, hkv, d, ldx, ld_qk, vt_ld, max_pos, NUL)


def test_qkv_rope_validation() -> None:
    check(*qkv()[:1], _lib.DX_ERR_INVALID, *qkv(first=NUL)[1:])
    check(*qkv()[:1], _lib.DX_ERR_UNSUPPORTED, *qkv(d=96)[1:])                  # head_dim not in {64,128,256}
    check(*qkv()[:1], _lib.DX_ERR_UNSUPPORTED, *qkv(hq=3, hkv=1, d=64)[1:])     # packed width 320
    check(*qkv()[:1], _lib.DX_ERR_UNSUPPORTED, *qkv(hidden=500, ldx=504)[1:])   # hidden % 64
    check(*qkv()[:1], _lib.DX_ERR_INVALID, *qkv(ld_qk=700)[1:])                 # below (hq + hkv) d
    check(*qkv()[:1], _lib.DX_OK, *qkv(rows=0)[1:])


def test_vt_zero_tails_validation() -> None:
    check("dx_vt_zero_tails", _lib.DX_ERR_INVALID, P, P, P, 2, 16, 60, NUL)       # vt_ld % 8
    check("dx_vt_zero_tails", _lib.DX_ERR_INVALID, NUL, P, P, 2, 16, 64, NUL)
    check("dx_vt_zero_tails", _lib.DX_OK, P, P, P, 0, 16, 64, NUL)


def test_head_op_validation() -> None:
    check("dx_linear_f32", _lib.DX_ERR_INVALID, P, P, NUL, P, 4, 8, 8, 8, 8, 8, _lib.DX_ACT_SILU, 0, NUL)
    check("dx_linear_f32", _lib.DX_ERR_INVALID, P, P, NUL, P, 4, 8, 8, 4, 8, 8, _lib.DX_ACT_NONE, 0, NUL)
    check("dx_linear_f32", _lib.DX_OK, P, P, NUL, P, 0, 8, 8, 8, 8, 8, _lib.DX_ACT_GELU_ERF, 1, NUL)
    check("dx_mha_f32", _lib.DX_ERR_UNSUPPORTED, P, P, P, P, P, 1, 4, 40000, 2, 8, 16, 16, 16, 16, NUL)
    check("dx_mha_f32", _lib.DX_ERR_INVALID, P, P, P, P, P, 1, 4, 64, 2, 8, 15, 16, 16, 16, NUL)
    check("dx_mha_f32", _lib.DX_OK, P, P, P, P, P, 1, 0, 64, 2, 8, 16, 16, 16, 16, NUL)
    check("dx_layer_norm_f32", _lib.DX_ERR_INVALID, P, P, NUL, P, 4, 16, 8, 16, ctypes.c_float(1e-5), NUL)
    check("dx_span_means_f32", _lib.DX_ERR_INVALID, P, P, P, 2, 0, 3, 16, 16, 16, NUL)
    check("dx_gather_rows_f32", _lib.DX_ERR_INVALID, P, P, P, 2, 0, 3, 16, 16, 16, 0, NUL)
    check("dx_head_routing_f32", _lib.DX_ERR_UNSUPPORTED, P, P, P, P, P, 1, 20000, 4, 16, NUL)
    check("dx_head_combine_f32", _lib.DX_OK, P, P, P, P, P, 0, ctypes.c_float(0.5), ctypes.c_float(2.0), NUL)


@pytest.mark.parametrize("name", sorted(_lib.SIGNATURES))
def test_every_entry_point_has_a_signature_bound(name: str) -> None:
    fn = getattr(lib(), name)
    restype, argtypes = _lib.SIGNATURES[name]
    assert fn.restype == restype and list(fn.argtypes) == list(argtypes)



def test_attention_grid_limits() -> None:
    """Counts beyond what a launch grid's y / z dimension holds are refused, not launched."""
    f = ctypes.c_float

    def vt(nseq, maxlen, hq=4, hkv=2):
        return status("dx_attn_prefill_vt", P, P, P, P, P, P, P, nseq, maxlen, hq, hkv, 128, 512, 256, 4096, 512,
                      f(0.1), f(50.0), 0, 1, NUL)

    for got in (vt(70000, 64), vt(4, 64, hq=140000, hkv=70000)):
        assert got == _lib.DX_ERR_UNSUPPORTED
        assert b"launch grid" in lib().dx_last_error()
    check("dx_transpose_v", _lib.DX_ERR_UNSUPPORTED, P, P, P, P, P, 70000, 64, 2, 128, 256, 4096, NUL)
    check("dx_transpose_v", _lib.DX_OK, P, P, P, P, P, 0, 64, 2, 128, 256, 4096, NUL)


def test_attention_32bit_ranges_refused() -> None:
    """The bf16 kernel's K and V^T buffer ranges are 32-bit: spans of 2 GiB or more are refused
    before any launch instead of wrapping."""
    f = ctypes.c_float

    def vt(maxlen, k_stride, vt_ld, d=256):
        return status("dx_attn_prefill_vt", P, P, P, P, P, P, P, 1, maxlen, 16, 8, d, 8192, k_stride, vt_ld, 4096,
                      f(0.0625), f(50.0), 0, 1, NUL)

    for args in ((16384, 1 << 16, 16384),    # 16384 keys x 64K-element rows = 2 GiB of K
                 (64, 2048, 1 << 23)):       # 255 x 8M-element V^T rows
        assert vt(*args) == _lib.DX_ERR_UNSUPPORTED
        assert b"2 GiB" in lib().dx_last_error()

    def packed(nseq, maxlen, d=256):
        return status("dx_attn_prefill", P, P, P, P, P, P, nseq, maxlen, 16, 8, d, 4096, 2048, 2048, 4096,
                      f(0.0625), f(50.0), 0, 1, _lib.DX_BF16, P, 1 << 40, NUL)

    # V^T of 2048 sequences x 4096 keys per KV head row: (D - 1) x 8M columns x 2 bytes > 2 GiB
    assert packed(2048, 4096) == _lib.DX_ERR_UNSUPPORTED
    assert b"2 GiB" in lib().dx_last_error()

    # fp32: a 32-key block of K or V is read through 32-bit byte offsets, so row strides stop at 2^24
    fp32 = status("dx_attn_prefill", P, P, P, P, P, P, 1, 64, 8, 4, 128, 1024, 1 << 24, 512, 1024,
                  f(0.088), f(0.0), 0, 1, _lib.DX_F32, NUL, 0, NUL)
    assert fp32 == _lib.DX_ERR_UNSUPPORTED and b"2^24" in lib().dx_last_error()
    # the limit is checked before an empty call returns, and only at head_dim 64 / 128: the head_dim 256
    # kernel addresses with 64-bit pointers, so the same strides pass (empty calls, no launch)
    def fp32_empty(d):
        return status("dx_attn_prefill", P, P, P, P, P, P, 0, 64, 8, 4, d, 8 * d, 1 << 24, 1 << 24, 8 * d,
                      f(0.0625), f(0.0), 0, 1, _lib.DX_F32, NUL, 0, NUL)

    assert fp32_empty(128) == _lib.DX_ERR_UNSUPPORTED
    assert fp32_empty(256) == _lib.DX_OK, lib().dx_last_error()


def test_noalloc_attention_refuses_oversize_before_any_launch() -> None:
    """dx_attn_prefill_noalloc stages V^T in a static scratch of DX_NOALLOC_SCRATCH_BYTES; a call that
    needs more is refused with DX_ERR_UNSUPPORTED before touching the device."""
    f = ctypes.c_float
    need = lib().dx_attn_prefill_workspace(64, 4096, 8, 256, _lib.DX_BF16)
    assert need > _lib.DX_NOALLOC_SCRATCH_BYTES
    got = status("dx_attn_prefill_noalloc", P, P, P, P, P, P, 64, 4096, 16, 8, 256, 4096, 2048, 2048, 4096,
                 f(0.0625), f(50.0), 0, 1, _lib.DX_BF16, NUL)
    assert got == _lib.DX_ERR_UNSUPPORTED
    assert b"static scratch" in lib().dx_last_error()
    check("dx_attn_prefill_noalloc", _lib.DX_OK, P, P, P, P, P, P, 0, 4096, 16, 8, 256, 4096, 2048, 2048, 4096,
          f(0.0625), f(50.0), 0, 1, _lib.DX_BF16, NUL)


def test_linear_residual_norm_validation() -> None:
    def lrn(m=8, d=512, k=256, lda=256, ldw=256, h=P, next_w=P, counters=P, post_w=P):
        return ("dx_linear_residual_norm", P, P, P, P, post_w, next_w, h, counters, m, d, k, lda, ldw, 1e-6, NUL)

    name = lrn()[0]
    check(name, _lib.DX_ERR_INVALID, *lrn(post_w=NUL)[1:])
    check(name, _lib.DX_ERR_INVALID, *lrn(counters=NUL)[1:])
    check(name, _lib.DX_ERR_INVALID, *lrn(h=NUL)[1:])                    # h without next_w's partner
    check(name, _lib.DX_ERR_UNSUPPORTED, *lrn(d=320)[1:])                # d % 256
    check(name, _lib.DX_ERR_UNSUPPORTED, *lrn(d=6400)[1:])               # d above 6144
    check(name, _lib.DX_ERR_UNSUPPORTED, *lrn(k=200, lda=200, ldw=200)[1:])
    check(name, _lib.DX_ERR_INVALID, *lrn(lda=128)[1:])                  # lda below k
    check(name, _lib.DX_ERR_INVALID, *lrn(counters=ctypes.c_void_p(0x10002))[1:])
    check(name, _lib.DX_OK, *lrn(m=0)[1:])
    check(name, _lib.DX_OK, *lrn(m=0, h=NUL, next_w=NUL)[1:])
    assert lib().dx_linear_residual_norm_counters(0) == 0
    assert lib().dx_linear_residual_norm_counters(70471) == (70471 + 255) // 256
    assert lib().dx_linear_residual_norm_counters(1000) == (1000 + 127) // 128


def test_readout_validation() -> None:
    """dx_readout refuses malformed sizes before any launch; option counts beyond the int32 range of the
    offsets are refused rather than truncated."""
    f = ctypes.c_float

    def ro(nq=2, nopt=6, rows=8, d=512, ld=512, vocab=100):
        return ("dx_readout", P, P, P, P, P, P, nq, nopt, rows, d, ld, vocab, f(1e-6), f(30.0), P, P, NUL)

    name = ro()[0]
    check(name, _lib.DX_ERR_INVALID, *ro(nopt=-1)[1:])
    check(name, _lib.DX_ERR_INVALID, *ro(nopt=1 << 31)[1:])
    check(name, _lib.DX_ERR_INVALID, *ro(rows=0)[1:])
    check(name, _lib.DX_ERR_INVALID, *ro(ld=256)[1:])
    check(name, _lib.DX_ERR_UNSUPPORTED, *ro(d=500, ld=504)[1:])
    check(name, _lib.DX_OK, *ro(nq=0)[1:])
