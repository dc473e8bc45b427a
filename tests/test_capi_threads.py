"""The C ABI's last-error text is per thread: calls refused at the same time on several host threads
(ctypes releases the GIL around each call) each read back their own message. Host-side only: every
call here is refused before any launch."""

import threading

from dllm_qwen38_amd import _lib

P = 1 << 16  # placeholder device address; refused calls never dereference it


def test_last_error_is_per_thread():
    L = _lib.lib()
    n_threads, reps = 6, 3000
    start = threading.Barrier(n_threads)
    bad = []

    def worker(i):
        length, block = 32 * (i + 1) + 16, 32  # a different refused length per thread
        want = f"L={length} is not a multiple of block={block}"
        start.wait()
        for _ in range(reps):
            st = L.dllm_fork_layout(1, length, block, 4, P, P, P, None)
            msg = _lib.last_error()
            if st != -1 or msg != want:
                bad.append((i, st, msg))
                return

    threads = [threading.Thread(target=worker, args=(i,)) for i in range(n_threads)]
    for t in threads:
        t.start()
    for t in threads:
        t.join()
    assert bad == []


def test_a_new_thread_starts_with_an_empty_message():
    L = _lib.lib()
    assert L.dllm_fork_layout(1, 48, 32, 4, P, P, P, None) == -1  # sets this thread's message
    seen = []
    t = threading.Thread(target=lambda: seen.append(_lib.last_error()))
    t.start()
    t.join()
    assert seen == [""]
    assert "not a multiple of block" in _lib.last_error()
