"""Hand-worked known-answer traces for the slab slot policy.

Each trace was worked by hand from the reference's text, not from either
implementation under test:

* decode steps: ExpertCache._begin(use_slab=True) (cache.py:2347-2453: clear
  pins, hit -> move_to_end + freq = min(8, freq + 1), pin; misses ->
  _alloc_slot :1118-1159), installs via _install -> _evict_to_budget
  (:2236-2291: while over budget, scan up to LFRU_SCAN entries from the LRU
  head, halving a positive freq and moving that entry to MRU, stopping at the
  first freq 0; then evict the first unpinned non-stitch entry from the head);
* prefill groups: _begin(prefill=True) with PREFILL_TOUCH=0 (:2367-2375: a hit
  is counted and nothing else), PREFILL_SLAB=1 (:2394-2401: misses take free
  slots with evict_ok=False), the stage for the rest (:2402-2411,
  _submit_stage :1392-1425) and _install(..., "soft") (:2306-2312: installed
  only while resident + 1 <= budget, else the slot is released);
* the free list is list(range(slots - 1, -1, -1)) popped from the end
  (:991, :1138-1139) and a released slot is appended (_release_slot :1116).

* flow decode: flow_admit (:861-910: clear pins; resident ids get MRU and
  reuse credit; other ids are misses and, unless their read is already in
  flight, take a slot with eviction allowed) and install on arrival
  (_attach_staging(install_now=True) :2866-2910 -> _install).

A policy adapter exposes: step(ids) -> [(miss id, slot)] (decode),
prefill(ids) -> (ticket, [(miss id, slot)], unplaced), done(ticket),
table() -> {expert: slot} of resident entries, evictions -> int.
"""

# 8 slots: reserve max(4, int(0.8)) = 4, budget 4.  Expert 0 is hit three
# times (freq 3).  Each later miss overfills the budget by one; when 0 is at
# the LRU head its counter halves 3 -> 1 -> 0 and it moves to MRU instead of
# being evicted; the third time (freq 0) it goes.  Plain LRU evicts it at
# step 8; a trim that never halves keeps it forever; one that halves but
# does not move it to MRU evicts it at step 8.
LFRU_SECOND_CHANCE = dict(
    slots=8,
    steps=[[0], [0], [0], [0], [1], [2], [3], [4], [5], [6], [7], [8], [9], [10], [11], [12]],
    # (step index, evicted experts in that step)
    evicted={7: [1], 8: [2], 9: [3], 10: [4], 11: [5], 12: [6], 13: [7], 14: [8], 15: [0]},
    # misses placed at each step: (expert, slot)
    placed={0: [(0, 0)], 4: [(1, 1)], 5: [(2, 2)], 6: [(3, 3)], 7: [(4, 4)], 8: [(5, 1)],
            9: [(6, 2)], 10: [(7, 3)], 11: [(8, 4)], 12: [(9, 1)], 13: [(10, 2)],
            14: [(11, 3)], 15: [(12, 4)]},
    final={9: 1, 10: 2, 11: 3, 12: 4},
)

# Same slab, plain LRU (lfru=False): expert 0 is the LRU head at step 8 and
# goes first, whatever its reuse count.
PLAIN_LRU = dict(
    slots=8,
    steps=LFRU_SECOND_CHANCE["steps"][:8],
    evicted={7: [0]},
    final={1: 1, 2: 2, 3: 3, 4: 4},   # 4 takes free slot 4; slot 0 returns to the free list
)

# Pins: hits and misses of the current step are not eviction candidates, so a
# step may leave the table over budget; the next step's trim brings it back.
# 8 slots, budget 4.  Step 1 installs 0..3 (slots 0..3).  Step 2 hits 0..3
# (freq 1 each, pinned) and misses 4 (slot 4, pinned): the scan halves 0..3
# to 0 and rotates them behind 4; every entry is pinned, nothing is evicted
# (5 resident).  Step 3 misses 5 (slot 5): pins are cleared, the head (4,
# freq 0) goes, then, still over budget, the new head 0 (freq 0) goes.
PINNED_OVER_BUDGET = dict(
    slots=8,
    steps=[[0, 1, 2, 3], [0, 1, 2, 3, 4], [5]],
    evicted={2: [4, 0]},
    placed={0: [(0, 0), (1, 1), (2, 2), (3, 3)], 1: [(4, 4)], 2: [(5, 5)]},
    final={1: 1, 2: 2, 3: 3, 5: 5},
)

# Prefill after a warm decode: 16 routed slots (reserve 4, budget 12) and an 8
# slot stage at slots 16..23.  Decode makes 0..11 resident (slots 0..11) and
# hits 0..3 twice (freq 2).  A prefill group over {0, 4, 20..25}: 0 and 4 are
# hits and keep their place; 20..23 take the four free slots 12..15 but the
# table is at budget, so they are held for the group only; 24, 25 take stage
# slots 16, 17.  No eviction.  After the group the four slots come back in
# order 12, 13, 14, 15, so the next decode miss (26) gets slot 15 and evicts
# the LRU head, 4 -- the hot set 0..3 survives.
PREFILL_AFTER_DECODE = dict(
    slots=16,
    stage=(16, 8),
    decode=[list(range(8)), list(range(8, 12)), [0, 1, 2, 3], [0, 1, 2, 3]],
    prefill=[0, 4, 20, 21, 22, 23, 24, 25],
    prefill_placed=[(20, 12), (21, 13), (22, 14), (23, 15), (24, 16), (25, 17)],
    compute_row={0: 0, 1: 1, 2: 2, 3: 3, 4: 4, 5: 5, 6: 6, 7: 7, 8: 8, 9: 9, 10: 10,
                 11: 11, 20: 12, 21: 13, 22: 14, 23: 15, 24: 16, 25: 17},
    after_prefill=dict(zip(range(12), range(12))),
    then_decode=[26],
    then_placed=[(26, 15)],
    then_evicted=[4],
)

# Prefill into a cold slab: misses are installed while the table is under
# budget (12), the rest held for the group.  16 slots, 14 misses: 0..11 are
# installed in slots 0..11, 12 and 13 use free slots 12 and 13 for the group
# only; after the group those two come back (free list [15, 14, 12, 13]).
PREFILL_COLD = dict(
    slots=16,
    stage=(16, 0),
    prefill=list(range(14)),
    prefill_placed=[(e, e) for e in range(14)],
    after_prefill=dict(zip(range(12), range(12))),
    then_decode=[30],
    then_placed=[(30, 13)],
    then_evicted=[0],
)


# Flow admission, 8 slots (budget 4).  Admit {0,1,2}: three misses, pending
# in slots 0..2, nothing resident.  Install them.  Admit {0,3}: 0 is a hit
# (MRU, freq 1), 3 a miss -> slot 3.  Admit {3} again before it lands: a miss,
# no second read.  Install 3 (4 resident).  Admit {4,5}: slots 4, 5.
# Install them: 4 makes 5 resident, the trim evicts the head 1 (freq 0); 5
# then evicts 2.  Final table {0:0, 3:3, 4:4, 5:5}; hits 1, misses 7.
FLOW_ADMIT = dict(
    slots=8,
    script=[("admit", [0, 1, 2], [(0, 0), (1, 1), (2, 2)]), ("install", [0, 1, 2]),
            ("admit", [0, 3], [(3, 3)]), ("admit", [3], []), ("install", [3]),
            ("admit", [4, 5], [(4, 4), (5, 5)]), ("install", [4, 5])],
    final={0: 0, 3: 3, 4: 4, 5: 5},
    hits=1, misses=7, evictions=2,
)


# Speculation, 16 slots (budget 12, free list [15, 14, 13, 12] once 0..11 are
# resident).  Guesses [20, 21, 5, 22, 23, 24] with at most 3 outstanding: 20,
# 21 take slots 12, 13; 5 is resident (skipped); 22 takes 14; the cap stops
# the rest.  A fetch of {20, 22, 30}: 20 and 22 are claimed (hits, no read),
# 30 misses into slot 15; installing 20, 22, 30 in id order evicts the LRU
# heads 0, 1, 2 (slots back to the free list in that order); the unclaimed
# guess 21 is handed back, and its slot 13 returns once its read has landed.
SPECULATION = dict(
    slots=16,
    warm=list(range(12)),
    guesses=[20, 21, 5, 22, 23, 24], max_staged=3,
    started=[(20, 12), (21, 13), (22, 14)],
    fetch=[20, 22, 30],
    fetch_placed=[(30, 15)],
    evicted=[0, 1, 2],
    hits=2, misses=12 + 1,
    free_after_settle=[0, 1, 2, 13],
)


def run_flow_kat(policy, kat):
    for op in kat["script"]:
        if op[0] == "admit":
            assert policy.admit(op[1]) == op[2], op
        else:
            policy.install(op[1])
    assert policy.table() == kat["final"], policy.table()
    assert (policy.hits, policy.misses, policy.evictions) == (kat["hits"], kat["misses"],
                                                              kat["evictions"])


def run_decode_kat(policy, kat):
    """Check a decode trace; returns the policy for further checks."""
    ev0 = policy.evictions
    for i, ids in enumerate(kat["steps"]):
        before = set(policy.table())
        placed = policy.step(ids)
        if "placed" in kat:
            assert placed == kat["placed"].get(i, []), (i, placed)
        after = set(policy.table())
        gone = sorted(before - after)
        want = kat["evicted"].get(i, [])
        assert gone == sorted(want), (i, gone, want)
    assert policy.table() == kat["final"], policy.table()
    assert policy.evictions - ev0 == sum(len(v) for v in kat["evicted"].values())
    return policy


def run_prefill_kat(policy, kat):
    for ids in kat.get("decode", []):
        policy.step(ids)
    ev0 = policy.evictions
    ticket, placed, unplaced = policy.prefill(kat["prefill"])
    assert placed == kat["prefill_placed"], placed
    assert unplaced == 0
    if "compute_row" in kat:
        assert policy.compute_row(ticket) == kat["compute_row"], policy.compute_row(ticket)
    assert policy.evictions == ev0, "a prefill group evicted"
    policy.done(ticket)
    assert policy.table() == kat["after_prefill"], policy.table()
    before = set(policy.table())
    placed = policy.step(kat["then_decode"])
    assert placed == kat["then_placed"], placed
    assert sorted(before - set(policy.table())) == kat["then_evicted"]
    return policy


# Prefill-time prediction (cache.py:2580-2650), 16 routed slots (budget 12)
# and a 6-slot stage at 16..21.  Decode makes layer 0's 0..9 resident (slots
# 0..9; free list [15, 14, 13, 12, 11, 10]).  prefill_ahead for layer 1,
# priority order [5, 3, 9, 1, 7, 2, 8], floors 2 and 2: 5, 3, 9, 1 take free
# slots 10..13 while more than 2 stay free; 7, 2, 8 take stage slots 16, 17,
# 18 while more than 2 stay in the stage.  Layer 1's prefill group over
# {1..6}: 1, 2, 3, 5 are claimed (hits, no read); 1 and 3 (routed slots) are
# installed while the table is under budget (10 -> 12), 2 (stage slot 17)
# and 5 (routed slot 10, table at budget) are held for the group; 4 and 6
# miss into free slots 14 and 15, held.  The unclaimed guesses 9, 7, 8 are
# handed back: once landed, slot 12 returns to the free list and 16, 18 to
# the stage; the group's own slots come back after it: free [12, 14, 10, 15].
PREFILL_AHEAD = dict(
    slots=16,
    stage=(16, 6),
    warm=list(range(10)),
    ahead=[5, 3, 9, 1, 7, 2, 8], free_floor=2, stage_floor=2,
    started=[(5, 10), (3, 11), (9, 12), (1, 13), (7, 16), (2, 17), (8, 18)],
    prefill=[1, 2, 3, 4, 5, 6],
    prefill_placed=[(4, 14), (6, 15)],
    compute_row={1: 13, 3: 11, 2: 17, 4: 14, 5: 10, 6: 15},
    after={1: 13, 3: 11},
    hits=4, misses=10 + 2, evictions=0,
    free_after=[12, 14, 10, 15],
    stage_after=[21, 20, 19, 16, 18, 17],
)
