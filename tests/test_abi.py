"""The C-ABI library loads, exports what include/okf_quant.h declares, and
validates arguments / injects faults on a detached (device -1) context.
No kernel runs here."""
import ctypes
import os
import re

import pytest

import chatokf_amd as ok

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def declared():
    text = open(os.path.join(ROOT, "include", "okf_quant.h")).read()
    return sorted(set(re.findall(r"^(?:int|const char \*)\s*(okf_\w+)\(", text, re.M)))


def test_header_declares_binding_exports():
    assert declared() == sorted(ok.EXPORTS)


def test_library_exports_every_declared_symbol():
    lib = ctypes.CDLL(ok.LIB_PATH)
    for name in declared():
        assert hasattr(lib, name), name


def test_row_bytes_abi():
    lib = ok.lib()
    out = ctypes.c_uint64()
    assert lib.okf_row_bytes(ok.Q4_K, 17408, ctypes.byref(out)) == 0 and out.value == 9792
    assert lib.okf_row_bytes(ok.IQ2_XXS, 5120, ctypes.byref(out)) == 0 and out.value == 1320
    assert lib.okf_row_bytes(ok.Q2_0, 6144, ctypes.byref(out)) == 0 and out.value == 1632
    assert lib.okf_row_bytes(ok.Q8_0, 2048, ctypes.byref(out)) == 0 and out.value == 2176
    assert lib.okf_row_bytes(ok.Q4_K, 100, ctypes.byref(out)) == ok.OKF_E_SHAPE
    assert lib.okf_row_bytes(ok.Q4_0, 64, ctypes.byref(out)) == 0 and out.value == 36
    assert lib.okf_row_bytes(3, 64, ctypes.byref(out)) == ok.OKF_E_TYPE  # Q4_1: not on this path


@pytest.fixture()
def detached():
    e = ok.Enc(-1)
    yield e
    e.close()


FAKE = 0x10000  # never dereferenced: a detached context launches nothing


def test_detached_context_validates_then_reports_nodev(detached):
    w = ok.QuantTensor(FAKE, 5120, 16, ok.Q4_K)
    with pytest.raises(ok.OkfError) as e:
        detached.gemv(w, FAKE, FAKE)
    assert e.value.status == ok.OKF_E_NODEV
    with pytest.raises(ok.OkfError) as e:
        detached.gemv(ok.QuantTensor(FAKE, 5000, 16, ok.Q4_K), FAKE, FAKE)
    assert e.value.status == ok.OKF_E_SHAPE
    with pytest.raises(ok.OkfError) as e:
        detached.gemv(ok.QuantTensor(FAKE, 5120, 16, 3), FAKE, FAKE)  # Q4_1: no kernel
    assert e.value.status == ok.OKF_E_TYPE
    with pytest.raises(ok.OkfError) as e:  # Q4_K wants 16-byte aligned blocks
        detached.gemv(ok.QuantTensor(FAKE + 8, 5120, 16, ok.Q4_K), FAKE, FAKE)
    assert e.value.status == ok.OKF_E_SHAPE
    with pytest.raises(ok.OkfError) as e:
        detached.gemm(w, FAKE, FAKE, 0)
    assert e.value.status == ok.OKF_E_SHAPE
    with pytest.raises(ok.OkfError) as e:
        detached.gemv(w, 0, FAKE)
    assert e.value.status == ok.OKF_E_ARG
    with pytest.raises(ok.OkfError) as e:
        detached.dequant_row(ok.QuantTensor(FAKE, 0, 0, ok.Q8_0), FAKE, 33)
    assert e.value.status == ok.OKF_E_SHAPE


def test_norm_and_argmax_validate_then_report_nodev(detached):
    cases = [
        (lambda: detached.add_rmsnorm(FAKE, FAKE, FAKE, FAKE, 2048, 1, 1e-6), ok.OKF_E_NODEV),
        (lambda: detached.add_rmsnorm(FAKE, None, FAKE, FAKE, 2048, 1, 1e-6), ok.OKF_E_NODEV),
        (lambda: detached.add_rmsnorm(None, FAKE, FAKE, FAKE, 2048, 1, 1e-6), ok.OKF_E_ARG),
        (lambda: detached.add_rmsnorm(FAKE, FAKE, FAKE, FAKE, 0, 1, 1e-6), ok.OKF_E_SHAPE),
        (lambda: detached.argmax_rows(FAKE, 248320, 1, FAKE), ok.OKF_E_NODEV),
        (lambda: detached.argmax_rows(FAKE, 0, 1, FAKE), ok.OKF_E_SHAPE),
        (lambda: detached.argmax_rows(FAKE, 16, 65536, FAKE), ok.OKF_E_SHAPE),
        (lambda: detached.argmax_rows(None, 16, 1, FAKE), ok.OKF_E_ARG),
    ]
    for call, status in cases:
        with pytest.raises(ok.OkfError) as e:
            call()
        assert e.value.status == status


def test_fault_injection_is_seeded(detached):
    # GPUGate.simulate analogue (LLM/Base/MetalGates.swift:101-108): with a
    # rate the calls fail with OKF_E_INJECTED, deterministically per seed.
    w = ok.QuantTensor(FAKE, 256, 4, ok.IQ2_XXS)

    def pattern(seed, rate, n=400):
        detached.set_fault_rate(rate, seed)
        out = []
        for _ in range(n):
            try:
                detached.gemv(w, FAKE, FAKE)
            except ok.OkfError as e:
                out.append(e.status == ok.OKF_E_INJECTED)
        return out

    a, b, c = pattern(7, 0.25), pattern(7, 0.25), pattern(8, 0.25)
    assert a == b and a != c
    assert 60 < sum(a) < 140
    assert sum(pattern(1, 0.0)) == 0
    assert sum(pattern(1, 1.0)) == 400
    with pytest.raises(ok.OkfError):
        detached.set_fault_rate(1.5, 0)


def test_bad_device_id():
    with pytest.raises(ok.OkfError):
        ok.Enc(-2)


def test_parallel_group_pairing(detached):
    # MetalEnc.parallel analogue: begin/end pair, no nesting
    lib, h = ok.lib(), detached.h
    assert lib.okf_parallel_end(h) == ok.OKF_E_ARG
    assert lib.okf_parallel_begin(h) == ok.OKF_OK
    assert lib.okf_parallel_begin(h) == ok.OKF_E_ARG
    # calls inside a group are validated when made
    with pytest.raises(ok.OkfError) as e:
        detached.gemv(ok.QuantTensor(FAKE, 5000, 16, ok.Q4_K), FAKE, FAKE)
    assert e.value.status == ok.OKF_E_SHAPE
    assert lib.okf_parallel_end(h) == ok.OKF_OK
    with detached.parallel():
        pass
