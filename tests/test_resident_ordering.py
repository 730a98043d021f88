"""Stream ordering of ResidentIndexUpdate.finish() (CPU, no device): which launches wait for
which events. The windowed prefetch's host copies run on their own stream and read each
prefetched token's host address and candidate slot when they run, so every launch that
rewrites those tables (the Index update, the LRU commit) or the slots they write (the Fetch
of the misses) must be ordered after the copies' event."""
import contextlib

from kvip_amd.operators.lifetch.resident import ResidentIndexUpdate


class Log:
    def __init__(self):
        self.entries = []


class FakeEvent:
    def __init__(self, log, name):
        self.log, self.name = log, name

    def record(self, stream):
        self.log.entries.append(("record", self.name, stream.name))


class FakeStream:
    def __init__(self, log, name):
        self.log, self.name, self.cuda_stream = log, name, name

    def wait_event(self, event):
        self.log.entries.append(("wait", event.name, self.name))


class FakeCuda:
    def __init__(self, log, main):
        self.log, self.main, self.current = log, main, main

    def current_stream(self, device=None):
        return self.current

    @contextlib.contextmanager
    def stream(self, s):
        saved, self.current = self.current, s
        try:
            yield
        finally:
            self.current = saved


class FakeTorch:
    def __init__(self, log, main):
        self.cuda = FakeCuda(log, main)


class FakeLibrary:
    def __init__(self, log):
        self.log = log

    def __getattr__(self, name):
        def launch(ref, stream):
            self.log.entries.append(("launch", name.replace("kvip_hip_resident_", ""), stream))
            return 0
        return launch


class FakeLru:
    def __init__(self, log, torch):
        self.log, self.torch = log, torch

    def commit(self, rows):
        self.log.entries.append(("launch", "lru_commit", self.torch.cuda.current_stream().name))


def make_update(overlap):
    log = Log()
    main = FakeStream(log, "main")
    torch = FakeTorch(log, main)
    upd = object.__new__(ResidentIndexUpdate)
    upd.torch, upd.library, upd.device, upd._ref = torch, FakeLibrary(log), "cuda:0", None
    upd.overlap = overlap
    upd.lru, upd.commit_rows = FakeLru(log, torch), None
    upd.after_resolve = None
    if overlap:
        upd.side = FakeStream(log, "side")
        upd.resolved, upd.updated = FakeEvent(log, "resolved"), FakeEvent(log, "updated")
    return upd, log


def position(entries, entry):
    assert entry in entries, (entry, entries)
    return entries.index(entry)


def ordered_after_copies(entries, launch_name):
    """True when the stream of `launch_name` waited for the copies' event before it."""
    stream = next(e[2] for e in entries if e[0] == "launch" and e[1] == launch_name)
    waits = [i for i, e in enumerate(entries) if e == ("wait", "copies_done", stream)]
    return bool(waits) and waits[0] < position(entries, ("launch", launch_name, stream))


def test_overlapped_finish_orders_update_and_lru_after_prefetch_copies():
    upd, log = make_update(overlap=True)
    upd.finish(copies_done=FakeEvent(log, "copies_done"))
    e = log.entries
    for name in ("update", "lru_commit", "fetch"):
        assert ordered_after_copies(e, name), (name, e)
    # The resolve needs only the decisions: it is not held back by the copies.
    assert position(e, ("launch", "resolve", "main")) < position(e, ("wait", "copies_done", "main"))
    # The update branch is forked after the resolve and joined after the Fetch.
    assert position(e, ("record", "resolved", "main")) < position(e, ("wait", "resolved", "side"))
    assert position(e, ("launch", "fetch", "main")) < position(e, ("wait", "updated", "main"))


def test_sequential_finish_orders_update_and_lru_after_prefetch_copies():
    upd, log = make_update(overlap=False)
    upd.finish(copies_done=FakeEvent(log, "copies_done"))
    e = log.entries
    for name in ("update", "lru_commit", "fetch"):
        assert ordered_after_copies(e, name), (name, e)


def test_finish_without_prefetch_copies_waits_for_nothing():
    upd, log = make_update(overlap=True)
    upd.finish()
    assert not any(x[0] == "wait" and x[1] == "copies_done" for x in log.entries)


def test_after_resolve_hook_runs_between_the_resolve_and_the_fetch():
    """A caller's fork point (MixedRound forks its prefill stage there): the hook sees the
    main stream right after the resolve is enqueued, before the Fetch, in both modes and
    with or without the prefetch copies."""
    for overlap in (True, False):
        for copies in (False, True):
            upd, log = make_update(overlap)
            upd.after_resolve = lambda stream, log=log: log.entries.append(("hook", stream.name))
            upd.finish(copies_done=FakeEvent(log, "copies_done") if copies else None)
            e = log.entries
            assert e.count(("hook", "main")) == 1, e
            hook = position(e, ("hook", "main"))
            assert position(e, ("launch", "resolve", "main")) < hook < position(e, ("launch", "fetch", "main")), e
