"""bench.py's host-side bookkeeping (no GPU): the launch-ceiling workload's
byte counts and the roofline traffic figure read from the committed counter
profile."""
import os
import sys

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
sys.path.insert(0, ROOT)

import bench  # noqa: E402


def test_ceiling_plan_matches_the_headline_token():
    """The ceiling workload reads exactly the headline token's algorithmic
    bytes (BASELINE config 3', 2,383,447,040 B for the Q4_K_M mix), in 113
    launches: four per layer and the lm_head."""
    plan = bench.token_launch_bytes("q4km")
    assert len(plan) == 4 * bench.LAYERS + 1
    assert sum(b for _, b, _ in plan) == 2_383_447_040
    assert sum(b for _, b, _ in bench.token_launch_bytes("q4k")) == 1_813_677_056
    # output bytes are the launches' y rows
    assert plan[-1] == ("lm_head", bench.VOCAB * (3072 // 256) * 144 + 4 * 3072 + 4 * bench.VOCAB,
                        4 * bench.VOCAB)


def test_roofline_traffic_comes_from_the_profile():
    t = bench.dominant_traffic_bytes("tiled")
    algo = 2 * bench.q4k_bytes(bench.FFN, bench.HIDDEN) + 4 * bench.HIDDEN + 8 * bench.FFN
    assert isinstance(t, int) and algo <= t <= 1.05 * algo
    assert bench.dominant_traffic_bytes("rows") is None
