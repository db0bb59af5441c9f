"""CPU checks of the C-ABI library: it loads without a GPU, exports every
symbol include/prime_mi355x.h declares, and rejects bad arguments before any
device work (error codes + prime_last_error)."""
import ctypes
import os
import re

import pytest

from prime_moment_attention import _lib

HDR = os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))), "include",
                   "prime_mi355x.h")


def _declared():
    src = open(HDR).read()
    return sorted(set(re.findall(r"^\s*(?:int|size_t|const char \*)\s*(prime_\w+)\s*\(", src, re.M)))


def test_header_declares_exports():
    assert _declared() == sorted(_lib.EXPORTS)


def test_library_loads_and_exports_every_symbol():
    L = _lib.load()
    for name in _declared():
        assert hasattr(L, name), name
    assert L.prime_abi_version() == _lib.ABI_VERSION


def test_null_arguments_rejected_without_device_work():
    L = _lib.load()
    st = _lib.PrimeState()
    rc = L.prime_decode_step(None, None, None, 1, 1, 1, 64, None, 1.0, None, ctypes.byref(st), None, None)
    assert rc == -1
    assert "null" in _lib.last_error()
    rc = L.prime_chunked_prefill(None, None, None, 1, 1, 1, 8, 64, 64, None, 1.0, 0, None, None, None, None, 0, None)
    assert rc == -1


def test_bad_dims_and_dtypes_rejected():
    L = _lib.load()
    t = _lib.PrimeTensor(16, _lib.PRIME_BF16, 0, 0, 0, 0)  # never dereferenced: validation fails first
    st = _lib.PrimeState(16, 16, 16, 16, 16, 16)
    b = ctypes.byref
    for D in (0, 65, 96, 128):  # 64, or 1 .. 63 (the token-sequential kernels)
        rc = L.prime_decode_step(b(t), b(t), b(t), 1, 1, 1, D, 16, 1.0, None, b(st), b(t), None)
        assert rc == -2 and "head dim" in _lib.last_error()
    rc = L.prime_decode_step(b(t), b(t), b(t), 1, 3, 2, 32, 16, 1.0, None, b(st), b(t), None)
    assert rc == -1  # head dim 32 is taken; H not a multiple of H_kv
    rc = L.prime_decode_step(b(t), b(t), b(t), 1, 3, 2, 64, 16, 1.0, None, b(st), b(t), None)
    assert rc == -1  # H not a multiple of H_kv
    t16 = _lib.PrimeTensor(16, _lib.PRIME_F16, 0, 0, 0, 0)
    rc = L.prime_chunked_prefill(b(t16), b(t16), b(t16), 1, 1, 1, 8, 64, 64, 16, 1.0, 0, None, b(t), None, None, 0, None)
    assert rc == -3
    rc = L.prime_chunked_prefill(b(t), b(t), b(t), 1, 1, 1, 8, 64, 64, 16, 1.0, 8, None, b(t), None, None, 0, None)
    assert rc == -1 and "flags" in _lib.last_error()
    tm = _lib.PrimeTensor(18, _lib.PRIME_BF16, 0, 0, 0, 0)  # misaligned rows
    rc = L.prime_chunked_prefill(b(tm), b(tm), b(tm), 1, 1, 1, 8, 64, 64, 16, 1.0, 0, None, b(tm), None, None, 0, None)
    assert rc == -4


def test_partial_state_overlap_rejected():
    L = _lib.load()
    t = _lib.PrimeTensor(16, _lib.PRIME_BF16, 0, 0, 0, 0)
    b = ctypes.byref
    base = 1 << 20
    sin = _lib.PrimeState(*[base + i * 65536 for i in range(6)])
    sout = _lib.PrimeState(*[base + (i + 6) * 65536 for i in range(5)] + [base + 5 * 65536])
    rc = L.prime_decode_step(b(t), b(t), b(t), 1, 1, 1, 64, 16, 1.0, b(sin), b(sout), b(t), None)
    assert rc == -5 and "overlaps" in _lib.last_error()


def test_gelu_and_delta_step_backward_validate_before_device_work():
    """prime_gelu and prime_delta_decode_step_backward reject null, misaligned,
    overlapping and out-of-range arguments with their error codes (no launch)."""
    L = _lib.load()
    assert L.prime_gelu(None, ctypes.c_void_p(16), 8, _lib.PRIME_BF16, None) == -1
    assert L.prime_gelu(ctypes.c_void_p(16), ctypes.c_void_p(16), -1, _lib.PRIME_BF16, None) == -1
    assert L.prime_gelu(ctypes.c_void_p(16), ctypes.c_void_p(16), 8, 9, None) == -3
    assert L.prime_gelu(ctypes.c_void_p(18), ctypes.c_void_p(48), 8, _lib.PRIME_BF16, None) == -4
    assert "aligned" in _lib.last_error()
    assert L.prime_gelu(ctypes.c_void_p(16), ctypes.c_void_p(32), 64, _lib.PRIME_BF16, None) == -5
    assert "overlaps" in _lib.last_error()
    assert L.prime_gelu(ctypes.c_void_p(16), ctypes.c_void_p(16), 0, _lib.PRIME_BF16, None) == 0  # nothing to do
    t = _lib.PrimeTensor(16, _lib.PRIME_BF16, 0, 0, 0, 0)
    b = ctypes.byref
    p = ctypes.c_void_p(4096)
    rc = L.prime_delta_decode_step_backward(b(t), b(t), b(t), p, p, 1, 1, 1, 64, 1e-5, 25.0, None, b(t), None,
                                            None, p, p, p, p, None, None)
    assert rc == -1 and "null" in _lib.last_error()
    rc = L.prime_delta_decode_step_backward(b(t), b(t), b(t), p, p, 1, 1, 1, 65, 1e-5, 25.0, None, b(t), None,
                                            p, p, p, p, p, None, None)
    assert rc == -2 and "head dim" in _lib.last_error()
    rc = L.prime_delta_decode_step_backward(b(t), b(t), b(t), p, p, 1, 3, 2, 64, 1e-5, 25.0, None, b(t), None,
                                            p, p, p, p, p, None, None)
    assert rc == -1  # H not a multiple of H_kv
    s_in = ctypes.c_void_p(1 << 20)
    rc = L.prime_delta_decode_step_backward(b(t), b(t), b(t), p, p, 1, 1, 1, 64, 1e-5, 25.0, s_in, b(t), None,
                                            p, p, p, p, p, ctypes.c_void_p((1 << 20) + 64), None)
    assert rc == -5 and "overlaps" in _lib.last_error()


def test_selective_log_decay_validates_before_device_work():
    """prime_selective_log_decay rejects null, out-of-range, misaligned and
    overlapping arguments with its error codes (no launch)."""
    L = _lib.load()
    st, tau, out = ctypes.c_void_p(1 << 20), ctypes.c_void_p(2 << 20), ctypes.c_void_p(3 << 20)
    bf = _lib.PRIME_BF16
    assert L.prime_selective_log_decay(None, bf, 24, 12, tau, 1e-4, 50.0, 2, 12, 8, out, None) == -1
    assert L.prime_selective_log_decay(st, bf, 96, 12, tau, 1e-4, 50.0, 2, 12, 0, out, None) == -1
    assert L.prime_selective_log_decay(st, bf, -1, 12, tau, 1e-4, 50.0, 2, 12, 8, out, None) == -1
    assert L.prime_selective_log_decay(st, 9, 96, 12, tau, 1e-4, 50.0, 2, 12, 8, out, None) == -3
    assert L.prime_selective_log_decay(st, bf, 96, 12, tau, 0.0, 50.0, 2, 12, 8, out, None) == -1
    assert "step bounds" in _lib.last_error()
    assert L.prime_selective_log_decay(st, bf, 96, 12, tau, 1.0, 0.5, 2, 12, 8, out, None) == -1
    assert L.prime_selective_log_decay(ctypes.c_void_p((1 << 20) + 1), bf, 96, 12, tau, 1e-4, 50.0, 2, 12, 8, out,
                                       None) == -4
    assert L.prime_selective_log_decay(st, bf, 96, 12, ctypes.c_void_p((2 << 20) + 2), 1e-4, 50.0, 2, 12, 8, out,
                                       None) == -4
    # out overlaps the pre-activations (2 x 8 rows of 12 bf16 from st)
    assert L.prime_selective_log_decay(st, bf, 96, 12, tau, 1e-4, 50.0, 2, 12, 8, ctypes.c_void_p((1 << 20) + 64),
                                       None) == -5
    assert "overlaps" in _lib.last_error()
    assert L.prime_selective_log_decay(st, bf, 96, 12, tau, 1e-4, 50.0, 2, 12, 8, ctypes.c_void_p((2 << 20) - 16),
                                       None) == -5  # out runs into tau


def test_host_wrappers_refuse_cpu_tensors():
    import torch
    x = torch.zeros(1, 1, 64)
    with pytest.raises(RuntimeError, match="HIP device"):
        _lib.decode_step(x, x, x, torch.ones(1), 1.0, None, _lib.new_state(1, 1, 64, "cpu"), x)


def test_workspace_plan():
    """Few long sequences are cut into segments (a workspace is requested);
    many sequences or the dense branch run one segment each (none needed)."""
    assert _lib.workspace_size(8, 12, 8192) > 0
    assert _lib.workspace_size(8, 12, 8192) % 16 == 0
    assert _lib.workspace_size(1, 1000, 8192) == 0
    assert _lib.workspace_size(8, 12, 8192, _lib.PRIME_FLAG_DENSE_CLAMP) == 0
    assert _lib.workspace_size(1, 1, 64) == 0


def test_timer_reads_without_launches():
    """The launch timer: an unknown kernel id is rejected; with nothing
    recorded every kernel reads zero launches (no device work involved)."""
    L = _lib.load()
    ms, n = ctypes.c_double(), ctypes.c_int64()
    assert L.prime_timer_read(len(_lib.KERNEL_NAMES), ctypes.byref(ms), ctypes.byref(n)) == -1
    assert L.prime_timer_read(0, None, None) == -1
    _lib.timer_enable()
    _lib.timer_reset()
    for kid in _lib.KERNEL_NAMES:
        assert _lib.timer_read(kid) == (0.0, 0)


def test_accumulate_noalloc_rejects_sizes_beyond_its_scratch():
    """prime_accumulate_noalloc needs one 33,792-byte slot per (sequence,
    head) in its fixed scratch: B * H = 993 is refused with a clear message
    before any device work (992 is the largest that fits)."""
    L = _lib.load()
    src = open(HDR).read()
    m = re.search(r"#define PRIME_NOALLOC_SCRATCH_BYTES \((\d+)u << (\d+)\)", src)
    assert m and int(m.group(1)) << int(m.group(2)) == _lib.NOALLOC_SCRATCH_BYTES
    assert _lib.NOALLOC_SCRATCH_BYTES // 33792 == 992
    t = _lib.PrimeTensor(16, _lib.PRIME_BF16, 0, 0, 0, 0)  # never dereferenced: validation fails first
    st = _lib.PrimeState(16, 16, 16, 16, 16, 16)
    b = ctypes.byref
    rc = L.prime_accumulate_noalloc(b(t), b(t), 3, 331, 331, 64, 64, 16, None, b(st), None)
    assert rc == -1
    msg = _lib.last_error()
    assert "993" in msg and "scratch" in msg and "prime_accumulate" in msg
    rc = L.prime_accumulate_noalloc(None, b(t), 1, 1, 1, 64, 64, 16, None, b(st), None)
    assert rc == -1 and "null" in _lib.last_error()
