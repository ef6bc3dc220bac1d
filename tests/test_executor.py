"""The CPU-task executor (include/naiwa_doorbell.h, src/executor.rs): one FIFO
worker, idle signalling, drain on close.  Host only."""
import threading
import time

from naiwa_moe.doorbells import Executor


def test_tasks_run_in_submission_order_on_one_worker():
    ex = Executor()
    seen, threads = [], set()
    for i in range(50):
        ex.submit(lambda i=i: (seen.append(i), threads.add(threading.get_ident())))
    ex.wait_idle()
    assert seen == list(range(50))
    assert len(threads) == 1 and threading.get_ident() not in threads
    assert ex.is_idle()
    ex.close()


def test_idle_only_after_the_running_task_finishes():
    ex = Executor()
    gate = threading.Event()
    ex.submit(lambda: gate.wait(5))
    time.sleep(0.05)
    assert not ex.is_idle()
    gate.set()
    ex.wait_idle()
    assert ex.is_idle()
    ex.close()


def test_close_drains_queued_tasks():
    ex = Executor()
    seen = []
    for i in range(10):
        ex.submit(lambda i=i: (time.sleep(0.002), seen.append(i)))
    ex.close()
    assert seen == list(range(10))
