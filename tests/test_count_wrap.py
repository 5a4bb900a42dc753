"""The contact sort after a count wrap and after a count the host sets, on the CPU oracle.

The reference sorts the first min(count, M) slots every substep (all_shaders.metal:711-745).
The GPU kernel skips the sort when no append reached a slot below M, since the list the last
sort left is then unchanged; these scenes are built so that skipping it at the wrong moment
gives a list different from the reference's:

  wrap          the count (a u32 no step clears, :765-766) is set 3 appends below 2^32; the
                remaining appends of the substep wrap to slots 0.. in the broad phase's
                (g, g') order, which for a body with two geoms is not pair-key order
  host count    slots a reset left behind (Q2 keeps the records) are exposed again by a count
                the host sets, on a step with no appends at all

tests/test_gpu_count_wrap.py runs the same scenes through the HIP step.
"""
import numpy as np

from oracle import oracle as O
from zeno_amd.model import load_model

# Body 1 carries two geoms, so its pairs with bodies 2 and 3 are appended as
# (g1,g3) (g1,g4) (g2,g3) (g2,g4): keys 12 13 12 13. No gravity: nothing moves.
INTERLEAVED = """<mujoco><option gravity="0 0 0"/><worldbody>{plane}
<body name="a" pos="0 0 0.5"><joint type="free"/><geom type="sphere" size="0.1" mass="1"/>
<geom type="sphere" size="0.1" pos="0.1 0 0" mass="1"/></body>
<body name="b" pos="0.2 0 0.5"><joint type="free"/><geom type="sphere" size="0.1" mass="1"/></body>
<body name="c" pos="0 0.2 0.5"><joint type="free"/><geom type="sphere" size="0.1" mass="1"/></body>
</worldbody></mujoco>"""
WITH_PLANE = INTERLEAVED.format(plane='<geom type="plane" size="5 5 0.1"/>')
NO_PLANE = INTERLEAVED.format(plane="")


def pair_key(a, b):
    return (min(a, b) << 16) | max(a, b)


def s1_appends(m, pos):
    """The broad phase's appends of one substep in (g, g') order, from its definition:
    different bodies, MuJoCo's contype/conaffinity rule, planes skip the distance test, other
    pairs need |c_a - c_b| < r_a + r_b + 0.1 (geom centre = body position + local offset)."""
    tb, ps = m["geoms"]["type_body"].astype(np.int64), m["geoms"]["pos_size0"].astype(np.float64)
    c = pos[tb[:, 1], :3].astype(np.float64) + ps[:, :3]
    out = []
    G = len(tb)
    for g in range(G):
        for o in range(g + 1, G):
            if tb[g, 1] == tb[o, 1]:
                continue
            if not ((tb[g, 3] & tb[o, 2]) or (tb[o, 3] & tb[g, 2])):
                continue
            if 3 not in (tb[g, 0], tb[o, 0]) and np.linalg.norm(c[o] - c[g]) >= ps[g, 3] + ps[o, 3] + 0.1:
                continue
            out.append((int(tb[g, 1]), int(tb[o, 1]), g, o))
    return out


def stable_by_key(pairs):
    return sorted(pairs, key=lambda p: pair_key(p[0], p[1]))


def test_appends_arrive_out_of_key_order():
    m = load_model(mjcf_string=WITH_PLANE)
    ap = s1_appends(m, m["init_positions"])
    assert len(ap) == 9
    assert stable_by_key(ap) != ap


def test_oracle_sorts_the_appends_after_the_wrap():
    """Count 2^32 - 3: the first three appends land beyond M, the last six wrap to slots 0-5.
    The reference's list is those six in stable key order; left in append order (the sort
    skipped at the wrap) it differs."""
    m = load_model(mjcf_string=WITH_PLANE)
    w = O.OracleWorld(m, 1)
    ap = s1_appends(m, m["init_positions"])
    w.contact_counts[:] = np.uint32(2**32 - 3)
    w.step(None)
    assert int(w.contact_counts[0]) == 6
    got = [tuple(int(v) for v in r) for r in w.contacts[0]["indices"][:6]]
    assert got == stable_by_key(ap[3:])
    assert got != ap[3:]


def stale_slot_sequence(world_like, m, reset_to_state, set_counts, step):
    """Step 1 with every body close (5 appends, sorted); a reset leaving only bodies 2 and 3
    close (one append, into slot 0, beside four stale slots); a reset with everything apart
    (counts 0, no appends); the host sets the count back to 5 and steps once."""
    p0, q0 = m["init_positions"], m["init_quaternions"]
    E = world_like
    pos = np.broadcast_to(p0, (E,) + p0.shape).astype(np.float32).copy()
    quat = np.broadcast_to(q0, (E,) + q0.shape).astype(np.float32).copy()
    step()
    near = pos.copy()
    near[:, 1, 0] -= 5.0
    reset_to_state(near, quat)
    step()
    far = near.copy()
    far[:, 3, 1] += 5.0
    reset_to_state(far, quat)
    set_counts(np.full(E, 5, np.uint32))
    step()


def test_oracle_sorts_slots_exposed_by_a_host_count():
    m = load_model(mjcf_string=NO_PLANE)
    w = O.OracleWorld(m, 1)
    seen = []

    def step():
        w.step(None)
        seen.append([tuple(int(v) for v in r) for r in w.contacts[0]["indices"][:5]])

    def set_counts(c):
        w.contact_counts[:] = c

    stale_slot_sequence(1, m, w.reset_to_state, set_counts, step)
    assert int(w.contact_counts[0]) == 5
    before = [seen[1][0]] + seen[0][1:]      # slot 0 rewritten by step 2, slots 1-4 from step 1
    assert [pair_key(a, b) for a, b, _, _ in before] != sorted(pair_key(a, b) for a, b, _, _ in before)
    assert seen[2] == stable_by_key(before)
