"""The ready map behind take_ready (nf4s_residency_*), on the CPU: the
prefetch state machine's take_ready loop (flowcast/src/state_machine.rs:
306-346) and FlowCastError::PrefetchMiss (flowcast/src/error.rs:20-25).
The table is host-only (no HIP call), so these run without a GPU; the
pinned pointers are plain host addresses the table never dereferences."""
import ctypes
import threading
import time

import pytest

from aethelstream_amd import _lib
from aethelstream_amd import stream as st

BUF = ctypes.create_string_buffer(64)
PTR = ctypes.addressof(BUF)


def _table(n):
    return st.Residency(n)


def test_deadline_checked_before_readiness():
    # state_machine.rs:309-313: the loop returns PrefetchMiss once
    # elapsed >= timeout, before looking at the ready map, so a zero timeout
    # misses even a resident layer; the layer stays resident.
    r = _table(4)
    r.publish(0, PTR, 64, st.PRECISION_NF4)
    with pytest.raises(st.PrefetchMiss, match="prefetch miss on layer 0") as e:
        r.wait(0, 0.0)
    assert e.value.layer_idx == 0
    assert r.wait(0, 0.01) == (PTR, 64, st.PRECISION_NF4)
    r.close()


def test_take_consumes_the_layer():
    # take_slot removes the slot (state_machine.rs:321-324): a second take
    # waits for the next publish.
    r = _table(2)
    r.publish(1, PTR, 10, st.PRECISIONS.index("INT4"))
    assert r.wait(1, 0.01) == (PTR, 10, st.PRECISIONS.index("INT4"))
    t0 = time.perf_counter()
    with pytest.raises(st.PrefetchMiss, match="prefetch miss on layer 1"):
        r.wait(1, 0.05)
    assert time.perf_counter() - t0 >= 0.045
    r.publish(1, PTR, 12, st.PRECISION_NF4)            # published again after the take
    assert r.wait(1, 0.01) == (PTR, 12, st.PRECISION_NF4)
    r.close()


def test_publish_from_another_thread_wakes_the_waiter():
    r = _table(3)

    def publisher():
        time.sleep(0.05)
        r.publish(2, PTR, 32, st.PRECISION_NF4)

    th = threading.Thread(target=publisher)
    t0 = time.perf_counter()
    th.start()
    got = r.wait(2, 5.0)                                 # the call releases the GIL
    dt = time.perf_counter() - t0
    th.join()
    assert got == (PTR, 32, st.PRECISION_NF4)
    assert 0.04 <= dt < 2.0, dt
    r.close()


def test_rejections():
    lib = _lib.load()
    r = _table(2)
    p, nb, pr = ctypes.c_void_p(), ctypes.c_int64(), ctypes.c_int32()
    rc = lib.nf4s_residency_wait(r.handle, 2, 1000, ctypes.byref(p), ctypes.byref(nb),
                                 ctypes.byref(pr))
    assert rc == 9 and b"beyond" in lib.nf4s_last_error_message()   # LAYER_NOT_FOUND
    assert lib.nf4s_residency_publish(r.handle, 5, PTR, 1, 5) == 9
    assert lib.nf4s_residency_publish(r.handle, 0, PTR, 1, 6) == 1    # unknown precision
    assert lib.nf4s_residency_publish(r.handle, 0, None, 1, 5) == 1   # NULL blob
    assert lib.nf4s_residency_publish(r.handle, 0, PTR, 1, 5) == 0
    assert lib.nf4s_residency_publish(r.handle, 0, PTR, 1, 5) == 1    # already resident
    assert b"already resident" in lib.nf4s_last_error_message()
    assert lib.nf4s_residency_wait(r.handle, 0, -1, ctypes.byref(p), ctypes.byref(nb),
                                   ctypes.byref(pr)) == 1              # negative timeout
    out = _lib.Nf4sReadyLayer()
    assert lib.nf4s_take_ready_wait(None, r.handle, 0, 1000, ctypes.byref(out)) == 1
    assert lib.nf4s_strerror(12) == b"prefetch miss"
    r.close()


def test_infinite_timeout_waits_for_the_publish():
    # float("inf") means "until published": the binding caps it at 10^9 s.
    r = _table(1)
    th = threading.Thread(target=lambda: (time.sleep(0.03), r.publish(0, PTR, 8, st.PRECISION_NF4)))
    th.start()
    assert r.wait(0, float("inf")) == (PTR, 8, st.PRECISION_NF4)
    th.join()
    with pytest.raises(_lib.Nf4sError, match="negative timeout"):
        r.wait(0, -1.0)
    r.close()


def test_huge_timeout_does_not_overflow_the_deadline():
    # INT64_MAX microseconds would overflow a nanosecond deadline; the table
    # clamps it, so a resident layer is still taken and not a miss.
    r = _table(1)
    r.publish(0, PTR, 4, st.PRECISION_NF4)
    lib = _lib.load()
    p, nb, pr = ctypes.c_void_p(), ctypes.c_int64(), ctypes.c_int32()
    assert lib.nf4s_residency_wait(r.handle, 0, 2**63 - 1, ctypes.byref(p), ctypes.byref(nb),
                                   ctypes.byref(pr)) == 0
    assert (p.value, nb.value) == (PTR, 4)
    r.close()
