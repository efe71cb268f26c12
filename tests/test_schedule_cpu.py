"""The continuous-batching plan (sr_go_tranformer_amd.schedule) against the
reference's own scheduler test (cmd/monolith/scheduler_test.go:18-58,
TestSchedulerTokenBudgetAndDecodeProgress) and the engine tick rules of
Engine.run (M:8370-8476)."""
from sr_go_tranformer_amd.schedule import TickPlanner, schedule_tokens


def test_scheduler_budget_and_decode_progress():
    # sessions: two decoding (cursor at the end of 2 and 3 ids), two with
    # 100-id prompts not started (scheduler_test.go:19-24)
    lens, cursor = [2, 3, 100, 100], [2, 2, 0, 0]
    remaining = [l - c for l, c in zip(lens, cursor)]
    extra = [0] * 4
    for tick in range(12):
        counts, total = schedule_tokens(remaining, 5, 4, 4, tick % 4)
        assert total == 5
        assert all(1 <= n <= 4 for n in counts)
        assert counts[0] == 1 and counts[1] == 1 and sum(counts) == total
        for i, n in enumerate(counts):
            extra[i] += n - 1
    assert extra[2] > 0 and extra[3] > 0
    counts, total = schedule_tokens(remaining, 1024, 16, 16, 0)
    assert total == 34 and counts[2] == 16 and counts[3] == 16
    # a decoding session caps prefill chunks at the mixed chunk
    counts, total = schedule_tokens(remaining, 64, 16, 1, 0)
    assert total == 4
    remaining[0] = 2  # sessions[0].Cursor = 0
    counts, total = schedule_tokens(remaining, 64, 16, 1, 0)
    assert total > 4


def test_round_robin_from_start():
    # 3 prefilling sessions, budget 4 -> one extra row, to session `start`
    for start in range(3):
        counts, total = schedule_tokens([10, 10, 10], 4, 16, 1, start)
        assert total == 4 and counts[start] == 2 and sum(counts) == 4


def test_tick_planner_follows_engine_ticks():
    prompts = [list(range(5)), list(range(40)), [7]]
    tp = TickPlanner(prompts, max_tokens=3, budget=8, chunk=4, mixed_chunk=1)
    trace = []
    step = 0
    while not tp.done():
        sessions, chunks, want = tp.plan()
        assert sum(len(c) for c in chunks) <= max(8, len(sessions))
        trace.append((sessions, [len(c) for c in chunks], want))
        tp.commit({s: 100 + step for s, w in zip(sessions, want) if w})
        step += 1
    # first tick: nobody decodes, budget 8 shared round-robin from rotation 0
    assert trace[0] == ([0, 1, 2], [4, 3, 1], [False, False, True])
    # session 2 (one-token prompt) samples on tick 0, then decodes: mixed
    # chunk 1 for everybody while it does
    assert trace[1][1] == [1, 1, 1]
    # every session ends with exactly max_tokens outputs
    assert all(len(o) == 3 for o in tp.outputs)
    # decode rows feed the previous output
    assert tp.outputs[2][0] == 100
