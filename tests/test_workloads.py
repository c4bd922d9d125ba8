"""The seeded workloads (CPU): the seeds chosen for a given first draw, and the
boundary batch's rows, whose draws the oracle must place exactly on, or one
uniform step beside, a step of the cumulative distribution."""
import numpy as np

from oracle import oracle as o
from promptboot_amd import workloads


def test_seed_for_draw_gives_that_first_draw():
    values = [0, 1, 2, 1 << 20, (1 << 23) - 1, 1 << 23, (1 << 24) - 1, 5_688_906]
    seeds = np.array([workloads.seed_for_draw(v, i) for i, v in enumerate(values)], np.uint64)
    assert workloads.next_24_stream(seeds).tolist() == values
    for v, sd in zip(values, seeds):  # and through the oracle's own generator
        st = o.SamplingState(int(sd))
        assert st.next_24() == v and st.draws() == 1


def test_boundary_rows_land_on_and_beside_the_steps():
    w = workloads.make("boundary", rows=128)
    tok, det, err, _ = o.sample_batch(w["logits"], w["hist"], w["hist_len"], w["random_24"],
                                      threads=8)
    assert (err["status"] == 0).all()
    assert (workloads.next_24_stream(w["seeds"]) == w["random_24"]).all()
    for r in range(128):
        kind, k = r % 4, (r // 4) % 16
        u = int(w["random_24"][r])
        if kind < 2:
            # 24-way tie: total 20, cutoff 16 on the 16th prefix, target 16 u
            assert det["kept"][r] == 16 and det["flags"][r] & 2
            step, off = divmod(u, 1 << 20)
            if off == 0:
                assert det["rank"][r] == step          # exactly on: the next survivor
            elif off == 1:
                assert det["rank"][r] == step
            else:
                assert off == (1 << 20) - 1 and det["rank"][r] == step  # just below step + 1
            assert kind == 0 and off == 0 or kind == 1 and off != 0
        elif kind == 2:
            assert det["kept"][r] == 2 and det["flags"][r] & 1
            assert det["rank"][r] == (0 if u < (1 << 23) else 1)
        else:
            assert det["flags"][r] == 0
