"""Several clips in flight on one GPU: a lane per clip, each on its own HIP stream.

The reference's benchmark loop runs one clip after another (runner.py:185-194) and each clip's decode
is a chain of small latency-bound launches that leaves most of the GPU idle. Here ``Scheduler`` keeps
``lanes`` decoders (``CustomModel.new_lane``: shared weights, private activations, caches, decoding
state and graphs) busy on separate streams. Each lane runs log-mel, the encoder graph and the prompt
steps, then 8-step decoder graph replays; after every replay an asynchronous copy of the token buffer
to pinned host memory and an event are enqueued, and the host polls the events instead of
synchronising, so a lane that waits for its tokens never stalls the others. Token ids are those of
``CustomModel.transcribe`` on the same clip (same kernels, same order on each lane's stream).
"""

import time

import torch

from .checkpoint import detokenize
from .config import CHUNK


class _Run:
    """One clip on one lane."""

    def __init__(self, index, max_new, stop_at_eos):
        self.index, self.max_new, self.stop_at_eos = index, max_new, stop_at_eos
        self.token_ids = None
        self.event = None
        self.start = time.perf_counter()
        self.ttft = None


class Scheduler:
    def __init__(self, model, lanes=2):
        if lanes < 1:
            raise ValueError('lanes must be >= 1')
        # One lane may be the model itself. Several lanes run concurrently, so each is a new lane with the
        # 32-launch decoder step: the persistent step needs every CU to itself.
        self.lanes = [model] if lanes == 1 else [model.new_lane() for _ in range(lanes)]
        self.streams = [torch.cuda.Stream() for _ in self.lanes]
        self.host_tokens = [torch.zeros(model.max_pos, dtype=torch.long, pin_memory=True) for _ in self.lanes]

    def _publish(self, li):
        """Token buffer -> pinned host copy, then an event; called on the lane's stream."""
        lane, stream = self.lanes[li], self.streams[li]
        self.host_tokens[li].copy_(lane.tokens, non_blocking=True)
        ev = torch.cuda.Event()
        ev.record(stream)
        return ev

    def _start(self, li, run, audio):
        lane = self.lanes[li]
        with torch.cuda.stream(self.streams[li]):
            lane._enqueue_mel(audio)
            lane._enqueue_encoder()
            lane._enqueue_prompt()
            run.event = self._publish(li)

    def _advance(self, li, run):
        """The lane's last event has completed: take its tokens; returns True when the clip is done."""
        lane, eos = self.lanes[li], self.lanes[li].eos
        host = self.host_tokens[li]
        if run.token_ids is None:
            run.token_ids = [int(host[0])]
            run.ttft = time.perf_counter() - run.start
        else:
            n = len(run.token_ids)
            for token in host[n:n + CHUNK].tolist():
                run.token_ids.append(token)
                if (run.stop_at_eos and token in eos) or len(run.token_ids) >= run.max_new:
                    break
        last = run.token_ids[-1]
        if (run.stop_at_eos and last in eos) or len(run.token_ids) >= run.max_new:
            return True
        with torch.cuda.stream(self.streams[li]):
            lane._replay(lane.graph_chunk, CHUNK)
            run.event = self._publish(li)
        return False

    @torch.inference_mode()
    def transcribe_many(self, clips, max_new_tokens=None, stop_at_eos=True):
        """Greedy token ids of every clip (same rules as CustomModel.transcribe), clips dealt to lanes as
        they free up. Returns one dict per clip with 'token_ids', 'text', 'ttft_s' and 'e2e_s' (seconds
        from this call's start), plus 'wall_s' of the whole batch in every dict."""
        budgets = [self.lanes[0]._check_audio(a, max_new_tokens) for a in clips]
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        pending = list(range(len(clips)))
        active = {}
        results = [None] * len(clips)
        while pending or active:
            for li in range(len(self.lanes)):
                if li not in active and pending:
                    idx = pending.pop(0)
                    run = _Run(idx, budgets[idx], stop_at_eos)
                    run.start = t0
                    self._start(li, run, clips[idx])
                    active[li] = run
            for li in list(active):
                run = active[li]
                if run.event.query() and self._advance(li, run):
                    lane = self.lanes[li]
                    fallback = False
                    if lane._step_fault():
                        # a persistent launch of this lane (the model itself, when it is the only lane)
                        # flagged a timed-out wait: its ids are not valid; transcribe decodes the clip
                        # again, falling back to the 34-launch step if it must
                        with torch.cuda.stream(self.streams[li]):
                            res = lane.transcribe(clips[run.index], run.max_new, stop_at_eos)
                        run.token_ids, fallback = res['token_ids'], True
                    results[run.index] = {'token_ids': run.token_ids, 'text': detokenize(lane.tokenizer, run.token_ids),
                                          'ttft_s': run.ttft, 'e2e_s': time.perf_counter() - t0,
                                          'n_tokens': len(run.token_ids), 'decode_fallback': fallback}
                    del active[li]
        torch.cuda.synchronize()
        wall = time.perf_counter() - t0
        for r in results:
            r['wall_s'] = wall
        return results
