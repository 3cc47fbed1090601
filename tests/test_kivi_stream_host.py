"""Host-side bookkeeping of the decode-time KIVI cache (no GPU): ring rows,
evicted blocks and window-old slots, against a brute-force model of the
token stream."""

from kivi_stream import RingState


def test_ring_bookkeeping_matches_token_model():
    R, G = 128, 32
    for n_groups in (0, 1, 4, 28):
        st = RingState(cap=R + G, residual=R, n_groups=n_groups, count=R)
        # token model: ring row of each token currently in the residual, and
        # the age order of window-old slots
        rows = list(range(R))          # tokens 0..R-1 of the prefill's residual
        slots = list(range(n_groups))  # oldest first
        for _ in range(5 * G + 7):
            row, blk, slot = st.append()
            assert row not in rows
            rows.append(row)
            if len(rows) == R + G:
                evicted = rows[:G]
                assert blk >= 0 and evicted == list(range(blk * G, blk * G + G))
                rows = rows[G:]
                if n_groups:
                    assert slot == slots[0]
                    slots = slots[1:] + slots[:1]
                else:
                    assert slot == -1
            else:
                assert blk == -1
            assert st.count == len(rows)
            assert [(st.start + i) % st.cap for i in range(st.count)] == rows
            assert not n_groups or [(st.next_slot + i) % n_groups for i in range(n_groups)] == slots


def _state_from_count(n, R, G, cap, n_groups):
    """The closed form kvdec_kivi_stream_step uses: the ring state after n
    appends, and the step taken by append n + 1."""
    e = n // G
    start, count = (G * e) % cap, R + n % G
    row = (start + count) % cap
    if count + 1 == cap:
        step = (row, start // G, e % n_groups if n_groups else -1)
        after = ((start + G) % cap, R)
    else:
        step = (row, -1, -1)
        after = (start, count + 1)
    return (start, count), step, after


def test_plan_closed_form_matches_ring_state():
    """The per-sequence step kernel derives each step from the append count
    alone; that closed form must agree with RingState.append() step by step."""
    R, G = 128, 32
    for n_groups in (0, 1, 4, 28):
        cap = R + G
        st = RingState(cap=cap, residual=R, n_groups=n_groups, count=R)
        for n in range(9 * G + 5):
            before, step, after = _state_from_count(n, R, G, cap, n_groups)
            assert before == (st.start, st.count), n
            row, blk, slot = st.append()
            assert step == (row, blk, slot if blk >= 0 else -1), n
            assert after == (st.start, st.count), n
