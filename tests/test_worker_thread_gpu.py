"""The reference's threaded launch contract on the drop-in mm_i8.

In the reference, prefill GEMMs are launched from a worker thread of their own
(pipeline.py:188-222): the thread first selects the accelerator for itself (use_npu,
pipeline.py:203-204), then runs one job at a time.  A job is a thunk that launches mm_i8 on a
slot buffer staged by the main thread (Prefill.gemm, pipeline.py:233-242; NPUGemm.stage /
launch_slot, gemma_npu.py:94-115).  The launch returns when C is ready; the worker records the
value, or the exception the launch raised, and wakes the scheduler, which consumes the result
on the main thread or re-raises the exception there (pipeline.py:212-216, 389-392).

The scheduler below is written for these tests: a condition-guarded job table, several slots
in flight, and the main thread restaging a slot's rows the moment its job is done while the
worker is still busy with other slots.  Results are checked bit for bit against torch._int_mm
on the host, the reference's CPU GEMM (pipeline.py:237).
"""
import collections
import threading

import pytest
import torch

import npu_kernels
from w8a8 import resident

pytestmark = pytest.mark.gpu


class Launcher:
    """One GEMM thread; run() hands back (job id, value or exception) of whichever job ends."""

    def __init__(self, stream=False):
        self._cv = threading.Condition()
        self._todo = collections.deque()
        self._ended = {}
        self._stop = False
        self.thread_ids = set()
        self._use_stream = stream
        self._t = threading.Thread(target=self._loop, daemon=True)
        self._t.start()

    def _loop(self):
        npu_kernels.use_npu()
        # The worker may launch on a stream of its own: mm_i8's completion must not depend on
        # the consumer sharing it.
        ctx = torch.cuda.stream(torch.cuda.Stream()) if self._use_stream else None
        if ctx is not None:
            ctx.__enter__()
        self.thread_ids.add(threading.get_ident())
        while True:
            with self._cv:
                while not self._todo and not self._stop:
                    self._cv.wait()
                if self._stop and not self._todo:
                    break
                jid, thunk = self._todo.popleft()
            try:
                out = thunk()
            except BaseException as e:  # noqa: BLE001 -- returned to the consumer
                out = e
            with self._cv:
                self._ended[jid] = out
                self._cv.notify_all()
        if ctx is not None:
            ctx.__exit__(None, None, None)

    def submit(self, jid, thunk):
        with self._cv:
            self._todo.append((jid, thunk))
            self._cv.notify_all()

    def next_done(self):
        with self._cv:
            while not self._ended:
                assert self._cv.wait(timeout=60), "worker did not finish a job within 60 s"
            jid = min(self._ended)
            out = self._ended.pop(jid)
        if isinstance(out, BaseException):
            raise out
        return jid, out

    def close(self):
        with self._cv:
            self._stop = True
            self._cv.notify_all()
        self._t.join(timeout=60)


class SlotGemm:
    """A static resident weight with per-slot staging rows and results, as NPUGemm keeps them
    (gemma_npu.py:57-115): stage(slot, T) gives the int8 rows to fill, launch(slot, T) runs
    mm_i8 on them and returns the [T, N] int32 view."""

    def __init__(self, w_nk, n_slots, rows, device=None):
        self.N, self.K = w_nk.shape
        self.w = resident.to_npu(w_nk.t().contiguous(), static=True)
        self.a = [resident.empty((rows, self.K), dtype=torch.int8, device=device) for _ in range(n_slots)]
        self.c = [resident.empty((rows, self.N), dtype=torch.int32, device=device) for _ in range(n_slots)]

    def stage(self, slot, T):
        return self.a[slot][:T]

    def launch(self, slot, T):
        return npu_kernels.mm_i8(self.a[slot][:T], self.w, self.c[slot][:T])


def _rows(seed, T, K):
    g = torch.Generator().manual_seed(seed)
    return torch.randint(-127, 128, (T, K), generator=g, dtype=torch.int8)


@pytest.mark.parametrize("where", ["host_slots", "device_slots", "device_slots_worker_stream"])
def test_worker_thread_runs_the_reference_call_pattern(where):
    K, N, rows, n_slots = 1536, 2560, 512, 4
    g = torch.Generator().manual_seed(7)
    w = torch.randint(-127, 128, (N, K), generator=g, dtype=torch.int8)
    wt = w.t().contiguous()
    dev = None if where == "host_slots" else "cuda"
    gemm = SlotGemm(w, n_slots, rows, device=dev)
    worker = Launcher(stream=where == "device_slots_worker_stream")
    # 12 micro-batches of ragged size through 4 slots; the main thread consumes on a stream of
    # its own, so nothing but mm_i8's completion orders its reads after the worker's GEMM.
    sizes = [512, 77, 512, 300, 1, 512, 129, 64, 512, 500, 33, 256]
    main_stream = torch.cuda.Stream()
    pending, expected, checked = {}, {}, 0
    with torch.cuda.stream(main_stream):
        free = list(range(n_slots))
        nxt = 0
        while nxt < len(sizes) or pending:
            while free and nxt < len(sizes):
                slot, T = free.pop(), sizes[nxt]
                xq = _rows(100 + nxt, T, K)
                gemm.stage(slot, T).copy_(xq)  # the main thread stages rows, pipeline.py:241
                expected[nxt] = torch._int_mm(xq, wt) if T > 16 else xq.int() @ wt.int()
                pending[nxt] = slot
                worker.submit(nxt, lambda s=slot, t=T: gemm.launch(s, t))
                nxt += 1
            jid, c = worker.next_done()
            slot = pending.pop(jid)
            got = c.cpu() if c.is_cuda else c.clone()
            assert torch.equal(got, expected.pop(jid)), f"micro-batch {jid} in slot {slot}"
            checked += 1
            # the slot is reused at once: staging overwrites rows the finished job read
            free.append(slot)
    worker.close()
    assert checked == len(sizes)
    assert threading.get_ident() not in worker.thread_ids, "the GEMMs must run on the worker thread"


def test_worker_exception_is_reraised_on_the_main_thread():
    """A shape error inside mm_i8 on the worker reaches the scheduler as the same exception
    (pipeline.py:212-213, 391-392), and the worker keeps serving later jobs."""
    K, N = 256, 64
    w = _rows(3, N, K)
    gemm = SlotGemm(w, 1, 64, device="cuda")
    worker = Launcher()
    bad_c = torch.empty((8, N + 1), dtype=torch.int32, device="cuda")
    worker.submit(0, lambda: npu_kernels.mm_i8(gemm.a[0][:8], gemm.w, bad_c))
    with pytest.raises(ValueError, match="mm_i8"):
        worker.next_done()
    worker.submit(1, lambda: npu_kernels.mm_i8(gemm.a[0][:8].cpu().float(), gemm.w, bad_c))
    with pytest.raises(TypeError, match="mm_i8"):
        worker.next_done()
    xq = _rows(4, 40, K)
    gemm.stage(0, 40).copy_(xq)
    worker.submit(2, lambda: gemm.launch(0, 40))
    jid, c = worker.next_done()
    assert jid == 2 and torch.equal(c.cpu(), torch._int_mm(xq, w.t().contiguous()))
    worker.close()


def test_host_rows_may_be_refilled_as_soon_as_mm_i8_returns():
    """Pinned host A with a device C: the rows are copied before mm_i8 returns, so refilling
    the staging buffer straight away cannot change the product."""
    K, N, T = 1536, 1024, 512
    w = _rows(5, N, K)
    pw = resident.to_npu(w.t().contiguous(), static=True)
    a = resident.empty((T, K), dtype=torch.int8)
    c = torch.empty((T, N), dtype=torch.int32, device="cuda")
    refs, outs = [], []
    for it in range(4):
        xq = _rows(10 + it, T, K)
        a.copy_(xq)
        npu_kernels.mm_i8(a, pw, c)
        a.fill_(127)  # the reference's next stage() overwrites the slot at once
        outs.append(c.clone())
        refs.append(torch._int_mm(xq, w.t().contiguous()))
    for it, (o, r) in enumerate(zip(outs, refs)):
        assert torch.equal(o.cpu(), r), f"iteration {it}"


def test_mm_i8_stream_ordered_when_asked():
    """wait=False: ordered on torch's current stream, consumed on that stream."""
    K, N, T = 512, 256, 100
    a = _rows(6, T, K)
    w = _rows(7, N, K)
    pw = resident.to_npu(w.t().contiguous(), static=True)
    c = torch.empty((T, N), dtype=torch.int32, device="cuda")
    s = torch.cuda.Stream()
    with torch.cuda.stream(s):
        npu_kernels.mm_i8(a.cuda(), pw, c, wait=False)
        got = c.cpu()
    assert torch.equal(got, torch._int_mm(a, w.t().contiguous()))
