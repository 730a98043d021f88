"""`kvip_amd.LIFetch(rotating, update)`: the graph-capturable decode round.

Keeps the reference's call shape (python/kvip/operators/lifetch/forward.py:7-17,
streaming.py:115-131): construction validates and packs every device address once;
``forward()`` takes no arguments, enqueues the round on the current stream and returns
None. The contiguous-Fetch forward is one C call; the resident forward is scoring + TopK
and then the round's resolve, with its Fetch beside the Index update on a second stream
joined before return (ResidentIndexUpdate(overlap=True)). It never allocates,
synchronises or reads back, so it can be captured into a hipGraph; argument problems
raise ValueError at construction, a failed launch raises RuntimeError.
"""
from __future__ import annotations

import ctypes

from kvip_amd.runtime import abi
from kvip_amd.operators.lifetch.binding import ContiguousFetch, LIFetchBinding
from kvip_amd.operators.lifetch.resident import ResidentIndexUpdate, ResidentPrefix


class LIFetchForward:
    """`update` is a ContiguousFetch (selected KV rows gathered into one buffer) or a
    ResidentIndexUpdate (hot-cache round: resolve, Fetch of the misses from host memory,
    Index update)."""

    def __init__(self, rotating, update, *, q_workers=2):
        """q_workers: the reference's per-request Fetch worker count
        (python/kvip/operators/lifetch/forward.py:8); accepted for call compatibility (a
        positive int). On MI355X the Fetch work is spread by the hardware dispatcher over
        every CU, so it selects nothing here."""
        if type(q_workers) is not int or q_workers < 1:
            raise ValueError(f"q_workers must be a positive int (got {q_workers!r})")
        self.q_workers = q_workers
        if not isinstance(rotating, LIFetchBinding):
            raise ValueError("LIFetch rotating must be a kvip_amd LIFetchBinding")
        if not isinstance(update, (ContiguousFetch, ResidentIndexUpdate)):
            raise ValueError("LIFetch update must be a kvip_amd ContiguousFetch or ResidentIndexUpdate")
        if update.rotating is not rotating:
            raise ValueError("Fetch destination was built for another LIFetch binding")
        if rotating.device != update.device:
            raise ValueError("Fetch and Index update must use the same device")
        self.rotating, self.update, self.torch = rotating, update, rotating.torch
        self.library = abi.load_library()
        self.set_options()
        # Called with the launch stream right after the round's scoring is enqueued; None:
        # nothing (the point from which a caller may fork work that should overlap the TopK
        # and what follows rather than the HBM-bound scoring).
        self.after_scoring = None
        self.resident = isinstance(update, ResidentIndexUpdate)
        if self.resident:
            self.indexer_args, self.topk_args = rotating.indexer_args(), rotating.topk_args()
            self.resident_args = update.args
            self._refs = (ctypes.byref(self.indexer_args), ctypes.byref(self.topk_args),
                          ctypes.byref(self.resident_args))
            self.prefix = None
            if update.prefetch is not None:
                torch = self.torch
                self.prefix = ResidentPrefix(torch, rotating, update.lru_slots, update.resident)
                pf = update.prefetch
                self.window_counts = torch.zeros((rotating.batch, abi.PREFETCH_MAX_WINDOWS), dtype=torch.int32,
                                                 device=rotating.device)
                self.prefetch_args = abi.PrefetchArgs(
                    victim_hits=abi.ptr(self.prefix.victim_hits), cold_hits=abi.ptr(self.prefix.cold_hits),
                    window_counts=abi.ptr(self.window_counts), cold_words=self.prefix.cold_words,
                    windows=pf.windows, window_limit=pf.window_limit, prefetch_limit=pf.prefetch_limit)
                self._prefetch_ref = ctypes.byref(self.prefetch_args)
                # The prefetch branch: its own stream (default priority), forked after the
                # scoring and joined before the final round.
                self.side = torch.cuda.Stream(device=rotating.device)
                self.scored, self.prefetched = torch.cuda.Event(), torch.cuda.Event()
                # Windowed prefetch (opt-in; fp8 scoring with one row per request): the
                # scoring runs window by window on the main stream; each scored window's cold
                # hits and prefetch decisions follow on the side stream and its host copies
                # on a third stream, so the copies overlap the scoring of later windows, the
                # final TopK, resolve and Index update; only the final Fetch waits for them.
                self.windowed = (pf.windowed and rotating.qk_name == "fp8" and rotating.rows_per_request == 1 and
                                 rotating.batch <= 512)
                if self.windowed:
                    self.copy = torch.cuda.Stream(device=rotating.device)
                    self.window_scored = [torch.cuda.Event() for _ in range(pf.windows)]
                    self.window_decided = [torch.cuda.Event() for _ in range(pf.windows)]
                    self.copies_done = torch.cuda.Event()
                    resident, history = update.resident, update.history
                    cold_tiles = (history - resident) // 128
                    # Scoring window e covers [bounds[e], bounds[e + 1]) (the last one runs to
                    # the row's end); prefetch window e >= 1 reads its cold hit words.
                    ends = [resident + 128 * (cold_tiles * e // max(1, pf.windows - 1)) for e in range(pf.windows)]
                    self.score_bounds = [0, resident] + ends[1:]
                    self.score_bounds[-1] = max(self.score_bounds[-1], rotating.key_stride)
                    self.hit_words = [None] + [((ends[e - 1] if e > 1 else resident) - resident) // 32
                                               for e in range(1, pf.windows)]
                    self.hit_words_end = [None] + [min((ends[e] - resident) // 32, self.prefix.cold_words)
                                                   for e in range(1, pf.windows)]
            return
        self.args = abi.LIFetchArgs(rotating.indexer_args(), rotating.topk_args(), update.fetch_args())
        self._args_ref = ctypes.byref(self.args)
        # Stage-wise argument blocks for score()/select()/fetch().
        self._indexer = ctypes.byref(self.args.indexer)
        self._topk = ctypes.byref(self.args.topk)
        self._fetch = ctypes.byref(self.args.fetch)
        # The forward's TopK: rows that fit the register-resident select take it even when
        # the split select's work memory is bound.
        self.topk_args = abi.TopkArgs.from_buffer_copy(self.args.topk)
        if self.topk_args.histogram and self.topk_args.key_stride <= abi.TOPK_REGS_MAX_KEYS:
            self.topk_args.segments = 0
        self._topk_fwd = ctypes.byref(self.topk_args)

    def set_options(self, *, diagnostics=False, deferred_fetch=False):
        """The reference's start-up option call (python/kvip/operators/lifetch/streaming.py:
        133-146, made with the defaults by forward.py:17 and by the test harness's
        set_deferred_fetch / set_diagnostics, tests/operators/lifetch/support/
        execution.py:3753-3757). Like the reference it touches no device memory and never
        runs inside forward().

        deferred_fetch: recorded and accepted either way. The reference packs it as bit 30 of
        its workspace option word, and no kernel of the reference reads that bit, so it
        changes no launched work there and none here.
        diagnostics: only False. True asks for the reference's in-kernel cycle stamps (bit
        31, read back through its `times` tensor), which this build does not record: per-
        kernel timings come from rocprofv3 and HIP events instead, so it raises ValueError
        rather than leaving a caller to read stamps that were never written."""
        if type(diagnostics) is not bool or type(deferred_fetch) is not bool:
            raise ValueError("set_options takes bool diagnostics and deferred_fetch")
        if diagnostics:
            raise ValueError("diagnostics=True: in-kernel cycle stamps are not recorded by this build "
                             "(profile the launches with rocprofv3 or HIP events)")
        self.diagnostics, self.deferred_fetch = diagnostics, deferred_fetch

    def _stream(self):
        return abi.stream_handle(self.torch, self.rotating.device)

    @property
    def plan(self):
        """The launch plan of a contiguous-Fetch forward: "three" (scoring, TopK, gather);
        "resident" for the resident-cache forward."""
        if self.resident:
            return "resident"
        code = self.library.kvip_hip_lifetch_plan(self._args_ref)
        if code not in abi.LIFETCH_PLANS:
            raise RuntimeError(f"LIFetch forward arguments rejected (code {code})")
        return abi.LIFETCH_PLANS[code]

    def __call__(self):
        if self.resident:
            upd = self.update
            if self.prefix is None:
                if not upd.overlap and upd.lru is None and self.after_scoring is None and upd.after_resolve is None:
                    abi.check(self.library.kvip_hip_resident_forward(*self._refs, self._stream()),
                              "resident LIFetch forward")
                    return
                # Scoring + round initialisation, TopK, then the round's resolve / Fetch /
                # Index update (the update beside the Fetch with overlap).
                abi.check(self.library.kvip_hip_resident_score(*self._refs, self._stream()), "resident scoring")
                self._scored()
                abi.check(self.library.kvip_hip_topk(self._refs[1], self._stream()), "TopK")
                upd.finish()
                return
            torch, lib = self.torch, self.library
            main = torch.cuda.current_stream(self.rotating.device)
            if self.windowed:
                self._windowed_prefetch_forward(torch, lib, main)
                return
            abi.check(lib.kvip_hip_resident_score(*self._refs, main.cuda_stream), "resident scoring")
            self._scored()
            self.scored.record(main)
            self.side.wait_event(self.scored)
            abi.check(lib.kvip_hip_resident_prefix(ctypes.byref(self.prefix.topk_args), ctypes.byref(self.prefix.args),
                                                   self.side.cuda_stream), "resident prefix")
            abi.check(lib.kvip_hip_resident_prefetch(self._refs[2], self._prefetch_ref, self.side.cuda_stream),
                      "resident prefetch")
            self.prefetched.record(self.side)
            abi.check(lib.kvip_hip_topk(self._refs[1], main.cuda_stream), "TopK")
            main.wait_event(self.prefetched)
            upd.finish()
            return
        if self.after_scoring is not None:
            self.score()
            self._scored()
            self.select()
            self.fetch()
            return
        abi.check(self.library.kvip_hip_lifetch_forward(self._args_ref, self._stream()), "LIFetch forward")

    def _scored(self):
        if self.after_scoring is not None:
            self.after_scoring(self.torch.cuda.current_stream(self.rotating.device))

    def _windowed_prefetch_forward(self, torch, lib, main):
        """The prefetching resident forward with the scoring in prefetch windows (same
        outputs as scoring first and prefetching after: every window's decisions see the
        same scores and run in window order)."""
        upd, pf = self.update, self.update.prefetch
        side, copy = self.side, self.copy
        bounds = self.score_bounds
        # Window 0: the resident prefix (with the round's initialisation); its TopK gives the
        # thresholds, then window 0's decisions (the victim candidates).
        abi.check(lib.kvip_hip_resident_score_window(*self._refs[:3], bounds[0], bounds[1], main.cuda_stream),
                  "resident scoring (prefix)")
        self.window_scored[0].record(main)
        side.wait_event(self.window_scored[0])
        abi.check(lib.kvip_hip_resident_threshold(ctypes.byref(self.prefix.topk_args), ctypes.byref(self.prefix.args),
                                                  side.cuda_stream), "resident threshold")
        for e in range(pf.windows):
            if e > 0:
                abi.check(lib.kvip_hip_indexer_decode_window(self._refs[0], bounds[e], bounds[e + 1],
                                                             main.cuda_stream), "resident scoring (window)")
                self.window_scored[e].record(main)
                side.wait_event(self.window_scored[e])
                if self.hit_words_end[e] > self.hit_words[e]:
                    abi.check(lib.kvip_hip_resident_cold_hits(ctypes.byref(self.prefix.args), self.hit_words[e],
                                                              self.hit_words_end[e], side.cuda_stream),
                              "resident cold hits")
            abi.check(lib.kvip_hip_resident_prefetch_windows(self._refs[2], self._prefetch_ref, e, e + 1,
                                                             side.cuda_stream), "resident prefetch decisions")
            self.window_decided[e].record(side)
            copy.wait_event(self.window_decided[e])
            abi.check(lib.kvip_hip_resident_prefetch_copy(self._refs[2], self._prefetch_ref, e, e + 1,
                                                          copy.cuda_stream), "resident prefetch copy")
        self.copies_done.record(copy)
        self._scored()
        abi.check(lib.kvip_hip_topk(self._refs[1], main.cuda_stream), "TopK")
        main.wait_event(self.window_decided[-1])
        upd.finish(copies_done=self.copies_done)

    # Individual stages (same kernels as the fused forward).
    def score(self):
        abi.check(self.library.kvip_hip_indexer_decode(self._indexer, self._stream()), "LI scoring")

    def select(self):
        abi.check(self.library.kvip_hip_topk(self._topk_fwd, self._stream()), "TopK")

    def fetch(self):
        abi.check(self.library.kvip_hip_fetch_gather(self._fetch, self._stream()), "Fetch gather")

    def select_fetch(self):
        """TopK fused with the Fetch gather in one launch (kvip_hip_select_fetch; needs the
        binding's segment work memory and rows of at most 32768 keys). Not part of the
        default forward, whose separate gather launch measured faster."""
        abi.check(self.library.kvip_hip_select_fetch(self._topk, self._fetch, self._stream()), "TopK+Fetch")
