"""Doorbell protocols and the CPU-task executor over include/naiwa_doorbell.h, with the
reference's class names and methods (src/doorbell/d2h/topk.rs, d2h/activation.rs,
h2d/result.rs, handoff.rs, src/executor.rs)."""
from __future__ import annotations

import ctypes as C

import numpy as np

from ._lib import RESULT_FN, TASK_FN, Pending, check, lib
from .ops import _dev


class _Handle:
    _destroy = ""

    def __del__(self):
        h = getattr(self, "_h", None)
        if h is not None and h.value:
            getattr(lib(), self._destroy)(h)
            self._h = C.c_void_p()


class TopkDoorbell(_Handle):
    _destroy = "naiwa_topk_doorbell_destroy"

    def __init__(self, max_n: int):
        self.max_n = max_n
        self._h = C.c_void_p()
        check(lib().naiwa_topk_doorbell_create(max_n, C.byref(self._h)), "topk_doorbell_create")

    def publish_and_read(self, ids, weights, n: int, stream: int = 0, timeout_us: int = 10_000_000):
        ids_out = np.empty(n, dtype=np.uint32)
        w_out = np.empty(n, dtype=np.float32)
        check(lib().naiwa_topk_doorbell_publish_and_read(self._h, _dev(ids), _dev(weights), n, stream,
                                                        ids_out.ctypes.data, w_out.ctypes.data, timeout_us),
              "topk_doorbell_publish_and_read")
        return ids_out, w_out


class ActivationDoorbell(_Handle):
    _destroy = "naiwa_act_doorbell_destroy"
    depth = 8

    def __init__(self, max_n: int):
        self.max_n = max_n
        self._h = C.c_void_p()
        check(lib().naiwa_act_doorbell_create(max_n, C.byref(self._h)), "act_doorbell_create")

    def publish(self, src, n: int, seq: int, stream: int = 0) -> None:
        check(lib().naiwa_act_doorbell_publish(self._h, _dev(src), n, seq, stream), "act_doorbell_publish")

    def wait_publish(self, seq: int, n: int, timeout_us: int = 250_000):
        out = np.empty(n, dtype=np.float32)
        found = C.c_int()
        check(lib().naiwa_act_doorbell_wait_publish(self._h, seq, n, out.ctypes.data, timeout_us, C.byref(found)),
              "act_doorbell_wait_publish")
        return out if found.value else None


class ResultDoorbell(_Handle):
    _destroy = "naiwa_result_doorbell_destroy"
    depth = 8

    def __init__(self, max_n: int):
        self._h = C.c_void_p()
        check(lib().naiwa_result_doorbell_create(max_n, C.byref(self._h)), "result_doorbell_create")

    @property
    def max_n(self) -> int:
        return lib().naiwa_result_doorbell_max_n(self._h)

    def publish(self, values, seq: int) -> bool:
        written = C.c_int()
        if values is None:
            check(lib().naiwa_result_doorbell_publish(self._h, None, 0, seq, C.byref(written)), "publish")
        else:
            v = np.ascontiguousarray(values, dtype=np.float32)
            check(lib().naiwa_result_doorbell_publish(self._h, v.ctypes.data, v.size, seq, C.byref(written)),
                  "publish")
        return bool(written.value)

    def wait_copy(self, seq: int, n: int, dst, stream: int = 0) -> None:
        check(lib().naiwa_result_doorbell_wait_copy(self._h, seq, n, _dev(dst), stream), "wait_copy")

    def consumed(self) -> int:
        c = C.c_uint32()
        check(lib().naiwa_result_doorbell_consumed(self._h, C.byref(c)), "consumed")
        return c.value


class PassCell(_Handle):
    _destroy = "naiwa_pass_cell_destroy"

    def __init__(self):
        self._h = C.c_void_p()
        check(lib().naiwa_pass_cell_create(C.byref(self._h)), "pass_cell_create")

    def claim(self, copy_stream: int) -> int:
        c = C.c_uint32()
        check(lib().naiwa_pass_cell_claim(self._h, copy_stream, C.byref(c)), "pass_cell_claim")
        return c.value

    def wait_latest(self, stream: int = 0) -> int | None:
        c = C.c_uint32()
        check(lib().naiwa_pass_cell_wait_latest(self._h, stream, C.byref(c)), "pass_cell_wait_latest")
        return c.value or None

    def claimed(self) -> int:
        c = C.c_uint32()
        check(lib().naiwa_pass_cell_claimed(self._h, C.byref(c)), "pass_cell_claimed")
        return c.value


class Executor(_Handle):
    """One FIFO worker thread; Python callables are kept alive until they ran."""
    _destroy = "naiwa_executor_destroy"

    def __init__(self):
        self._h = C.c_void_p()
        self._keep = []
        check(lib().naiwa_executor_create(C.byref(self._h)), "executor_create")

    def submit(self, fn) -> None:
        cb = TASK_FN(lambda _u: fn())
        self._keep.append(cb)
        check(lib().naiwa_executor_submit(self._h, cb, None), "executor_submit")

    def is_idle(self) -> bool:
        return lib().naiwa_executor_is_idle(self._h) == 1

    def wait_idle(self, timeout_us: int = 10_000_000) -> None:
        check(lib().naiwa_executor_wait_idle(self._h, timeout_us), "executor_wait_idle")

    def submit_result(self, n: int, compute) -> Pending:
        """compute() -> n float32 values, run on the worker; raising counts as a failure."""
        def run(_u, out, length):
            try:
                v = np.asarray(compute(), dtype=np.float32).reshape(-1)
                if v.size != length:
                    return 2
                C.memmove(out, v.ctypes.data, v.nbytes)
                return 0
            except Exception:
                return 1
        cb = RESULT_FN(run)
        self._keep.append(cb)
        p = Pending()
        check(lib().naiwa_executor_submit_result(self._h, n, cb, None, C.byref(p)), "executor_submit_result")
        return p

    def upload(self, pending: Pending, dst, stream: int = 0) -> None:
        check(lib().naiwa_pending_upload(self._h, C.byref(pending), _dev(dst), stream), "pending_upload")

    def take_error(self) -> str | None:
        buf = C.create_string_buffer(256)
        rc = lib().naiwa_executor_take_error(self._h, buf, 256)
        return buf.value.decode() if rc else None

    def stalls(self) -> int:
        s = C.c_uint64()
        check(lib().naiwa_executor_stalls(self._h, C.byref(s)), "executor_stalls")
        return s.value

    def close(self) -> None:
        if self._h.value:
            lib().naiwa_executor_destroy(self._h)
            self._h = C.c_void_p()
        self._keep.clear()


__all__ = ["TopkDoorbell", "ActivationDoorbell", "ResultDoorbell", "PassCell", "Executor"]
