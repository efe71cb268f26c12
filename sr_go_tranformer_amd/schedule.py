"""Host-side continuous-batching plan: the reference engine's scheduleTokens
and its per-tick session bookkeeping (cmd/monolith/monolith.go,
Engine.run M:8211-8476).  The engine actor itself (queues, HTTP, streaming)
stays in the Go caller; this restates the part that decides which rows each
step (prefillSelected, here srq_step) carries, so a driver of the C ABI
produces the same steps the reference engine would.
"""


def schedule_tokens(remaining, budget, chunk, mixed_chunk, start):
    """scheduleTokens (M:8180-8210).  remaining[i] = prompt tokens session i
    has not prefilled yet (0: it is decoding).  Every session gets one row;
    extra prefill rows go round-robin from `start`, each session up to
    min(chunk, remaining), until `budget` rows; while any session decodes the
    chunk is capped at mixed_chunk.  Returns (counts, total)."""
    n = len(remaining)
    if any(r == 0 for r in remaining):
        chunk = min(chunk, mixed_chunk)
    counts = [1] * n
    total = n
    while total < budget:
        progress = False
        for j in range(n):
            i = (start + j) % n
            if counts[i] < min(chunk, remaining[i]):
                counts[i] += 1
                total += 1
                progress = True
                if total == budget:
                    break
        if not progress:
            break
    return counts, total


class TickPlanner:
    """Engine.run's ticks (M:8370-8476) for requests admitted together, in
    request order: each tick schedules the live sessions (rotation advances
    by one per tick, modulo the live count), prefilling sessions send their
    next prompt rows and want logits once the prompt is complete, decoding
    sessions send their last output.  After the step, prefill cursors
    advance and every session that wanted logits receives one sampled token;
    a session leaves once it holds max_tokens outputs (or emits eos)."""

    def __init__(self, prompts, max_tokens, budget=64, chunk=16, mixed_chunk=1, eos=None):
        self.prompts = [list(p) for p in prompts]
        self.max_tokens = max_tokens
        self.budget, self.chunk, self.mixed_chunk, self.eos = budget, chunk, mixed_chunk, eos
        self.cursor = [0] * len(prompts)
        self.outputs = [[] for _ in prompts]
        self.live = list(range(len(prompts)))
        self.rotation = 0
        self.ticks = 0
        self._plan = None

    def done(self):
        return not self.live

    def plan(self):
        """The next step: (sessions, chunks, want) over the live sessions."""
        n = len(self.live)
        remaining = [len(self.prompts[i]) - self.cursor[i] for i in self.live]
        counts, _ = schedule_tokens(remaining, self.budget, self.chunk, self.mixed_chunk, self.rotation % n)
        self.rotation = (self.rotation + 1) % n
        chunks, want = [], []
        for k, i in enumerate(self.live):
            c = self.cursor[i]
            if c < len(self.prompts[i]):
                chunks.append(self.prompts[i][c:c + counts[k]])
            else:
                chunks.append([self.outputs[i][-1]])
            want.append(c + counts[k] >= len(self.prompts[i]))
        self._plan = (list(self.live), chunks, want)
        return self._plan

    def commit(self, sampled):
        """sampled: {session: token} for every planned session with want."""
        sessions, chunks, want = self._plan
        alive = []
        for k, i in enumerate(sessions):
            if self.cursor[i] < len(self.prompts[i]):
                self.cursor[i] += len(chunks[k])
            if self.cursor[i] < len(self.prompts[i]):
                alive.append(i)
                continue
            tok = sampled[i]
            self.outputs[i].append(tok)
            if (self.eos is not None and tok == self.eos) or len(self.outputs[i]) == self.max_tokens:
                continue
            alive.append(i)
        self.live = alive
        self.ticks += 1
        self._plan = None
