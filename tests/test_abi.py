"""The C-ABI library without a GPU: it loads, exports every symbol include/rvmoe.h declares
(and the Python view declares the same set), and its host-only entry points behave. No kernel
is launched here."""
import os
import re

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def header_functions():
    text = open(os.path.join(ROOT, "include", "rvmoe.h")).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"^\s*(?:const\s+)?\w+\s*\*?\s*(rv[hm]_\w+)\s*\(", text, flags=re.M)))


def test_header_declares_the_reference_runtime_and_moe_entry_points():
    names = header_functions()
    # the runtime, memory and event symbols of the reference's runtime/hip/rvhip.h:22-38
    for n in ["rvh_init", "rvh_mem_info", "rvh_alloc", "rvh_free", "rvh_upload", "rvh_download", "rvh_copy",
              "rvh_sync", "rvh_error_string", "rvh_event_create", "rvh_event_destroy", "rvh_event_record",
              "rvh_event_sync", "rvh_event_elapsed"]:
        assert n in names
    # the reference's expert-path kernels (rvhip.h:42-80)
    for n in ["rvh_rms_norm", "rvh_f32_mm", "rvh_q4_mm", "rvh_q4_mv", "rvh_geglu_split", "rvh_gather_rows",
              "rvh_moe_combine"]:
        assert n in names
    assert "rvm_moe_decode" in names and "rvm_moe_forward" in names


def test_library_exports_every_declared_symbol(rvlib):
    from rosevine_amd import hip
    names = header_functions()
    for n in names:
        assert hasattr(rvlib, n), n
    assert sorted(hip.SIGNATURES) == names


def test_host_generator_is_deterministic_and_shaped(rvlib):
    from rosevine_amd import hip
    a = hip.synth_q4_host(2, 64, 256, 7, 100)
    b = hip.synth_q4_host(2, 64, 256, 7, 100)
    c = hip.synth_q4_host(1, 64, 256, 7, 101)  # matrix 1 of the first stack = stream 101
    assert np.array_equal(a, b)
    assert np.array_equal(a[a.size // 2:], c)
    d = a.reshape(-1, 18)[:, :2].copy().view(np.float16).astype(np.float32).reshape(-1)
    assert d.min() >= np.float16(0.005) and d.max() <= np.float16(0.02)
    nib = a.reshape(-1, 18)[:, 2:]
    assert abs(float(nib.mean()) - 127.5) < 2.0


def test_packed_bytes_and_scalar_validation(rvlib):
    from rosevine_amd import hip
    assert hip.q4_packed_bytes(128, 1408, 2816, hip.PACK_GATE_UP) == 128 * 1408 * 88 * 18
    assert hip.q4_packed_bytes(128, 2816, 704, hip.PACK_ROWS32) == 128 * 2816 * 22 * 18
    for args in [(1, 1408, 2816, 7), (1, 1400, 2816, hip.PACK_GATE_UP), (1, 2816, 32, hip.PACK_ROWS32),
                 (0, 64, 64, hip.PACK_GATE_UP)]:
        try:
            hip.q4_packed_bytes(*args)
        except hip.DeviceError as e:
            assert e.code == 1  # hipErrorInvalidValue
        else:
            raise AssertionError(f"accepted {args}")


def test_bounds_are_checked_before_any_call(rvlib):
    from rosevine_amd import hip

    class Fake(hip.DevBuf):
        def __init__(self, n):  # no allocation: only the range logic is exercised
            self.ptr, self.nbytes = 0x1000, n

        def close(self):
            self.ptr = None

    w, x, y = Fake(100), Fake(4 * 2816), Fake(4 * 1408)
    try:
        hip.q4q8_mm(w, hip.PACK_GATE_UP, x, y, 1408, 2816, 1)
    except hip.BoundsError:
        pass
    else:
        raise AssertionError("out-of-allocation range accepted")


def test_phase_trace_only_in_the_diagnostic_build(rvlib):
    """The normal build compiles the decode kernels' phase stamps out: rvm_phase_trace refuses a
    short buffer and otherwise reports hipErrorNotSupported, with no device call."""
    buf = np.zeros(3 * 4096 * 8, np.uint64)
    assert rvlib.rvm_phase_trace(buf.ctypes.data, buf.nbytes - 8) != 0
    assert rvlib.rvm_phase_trace(buf.ctypes.data, buf.nbytes) == 801  # hipErrorNotSupported
    assert not buf.any()


def test_q4_mm_n_rejects_bad_counts_before_any_call(rvlib):
    """rvm_q4_mm_n validates its matrix count and arrays on the host (no device call is made)."""
    import ctypes as C
    w = (C.c_void_p * 5)(*([0x1000] * 5))
    y = (C.c_void_p * 5)(*([0x2000] * 5))
    rows = (C.c_int * 5)(*([64] * 5))
    for n in (0, 5):
        assert rvlib.rvm_q4_mm_n(n, w, rows, y, C.c_void_p(0x3000), 2816, 1) == 1  # hipErrorInvalidValue
    odd = (C.c_void_p * 2)(0x1000, 0x1001)  # a matrix that is not 2-byte aligned
    assert rvlib.rvm_q4_mm_n(2, odd, rows, y, C.c_void_p(0x3000), 2816, 1) == 1
    bad_rows = (C.c_int * 2)(64, 0)
    assert rvlib.rvm_q4_mm_n(2, w, bad_rows, y, C.c_void_p(0x3000), 2816, 1) == 1


def test_session_layer_ranges_are_refused_before_any_call(rvlib):
    """rvm_session_eval_range's contract (the cancellation points of runtime/src/hip_exec.rs:645-655):
    a range lies inside the stack, a range after layer 0 continues the evaluation in progress with the
    same tokens, layer 0 needs x and the last layer needs out. The Python host side makes the library's
    checks first, so none of these reaches the device; the library refuses a null session itself."""
    import pytest

    from rosevine_amd import hip, session

    class Buf(hip.DevBuf):
        def __init__(self, n):  # no allocation: only the range logic is exercised
            self.ptr, self.nbytes = 0x1000, n

        def close(self):
            self.ptr = None

    s = object.__new__(session.Session)
    s.layers, s.max_tokens, s.d, s.handle = [object()] * 4, 2, 256, None
    x, out = Buf(2 * 256 * 4), Buf(2 * 256 * 4)
    for l0, l1 in [(-1, 2), (2, 2), (3, 1), (0, 5), (4, 4)]:
        with pytest.raises(hip.BoundsError):
            s.eval_range(x, out, 1, l0, l1)
    with pytest.raises(hip.BoundsError):
        s.eval_range(x, out, 3, 0, 2)  # more tokens than the session holds
    with pytest.raises(hip.BoundsError):
        s.eval_range(None, out, 1, 0, 2)  # layer 0 reads x
    with pytest.raises(hip.BoundsError):
        s.eval_range(x, None, 1, 0, 4)  # the last layer writes out
    with pytest.raises(hip.BoundsError):
        s.eval_range(x, out, 1, 2, 4)  # no evaluation in progress: must start at layer 0
    s._next, s._ntok = 2, 1
    with pytest.raises(hip.BoundsError):
        s.eval_range(x, out, 1, 3, 4)  # does not continue at layer 2
    with pytest.raises(hip.BoundsError):
        s.eval_range(x, out, 2, 2, 4)  # other tokens than the evaluation in progress
    assert rvlib.rvm_session_eval_range(None, None, None, 1, 0, 0, 1) == 1  # hipErrorInvalidValue
    assert rvlib.rvm_session_probe(None, None, 0) == 1
