"""D-LSA K1 select oracle (oracle.dlsa_select) against the reference's golden
fixtures (tests/fixtures/dlsa: tiny, tiny_ties, qwen_layer random/real maps,
qwen_index_defaults = the served defaults, lists of 4,612): picked buckets and
read lists bit for bit. CPU only."""
import json
import os

import numpy as np
import pytest

from conftest import ROOT

GOLD = os.path.join(ROOT, "tests", "golden", "dlsa_select.safetensors")


def _cases():
    from safetensors import safe_open

    with safe_open(GOLD, framework="numpy") as f:
        meta = json.loads(f.metadata()["cases"])
        out = {}
        for tag, m in meta.items():
            t = {name: f.get_tensor(f"{tag}.{name}") for name in
                 ("bucket_scores", "bucket_members", "visible_buckets", "picked_buckets",
                  "selected", "selected_lengths", "positions")}
            out[tag] = (m["config"], t)
    return out


CASES = _cases()


def select_args(cfg, t):
    rows = t["bucket_scores"].shape[1]
    return dict(total_rows=rows, window=cfg["window_size"], sink=cfg["sink_size"],
                top_k=cfg["top_k"], top_p=cfg["top_p"],
                buckets_per_block=cfg["window_size"] // cfg["bucket_size"])


@pytest.mark.parametrize("tag", sorted(CASES))
def test_oracle_select_matches_fixtures(oracle_lib, tag):
    cfg, t = CASES[tag]
    lists, lengths, picked, status = oracle_lib.dlsa_select(
        t["bucket_scores"], t["bucket_members"], t["positions"], **select_args(cfg, t))
    args = select_args(cfg, t)
    vis = np.minimum(t["positions"] // args["window"] * args["buckets_per_block"],
                     args["total_rows"])
    assert np.array_equal(vis, t["visible_buckets"])
    assert not status.any()
    assert np.array_equal(picked, t["picked_buckets"])
    assert np.array_equal(lengths, t["selected_lengths"])
    assert np.array_equal(lists, t["selected"])


def test_oracle_select_nan_and_short_scores(oracle_lib):
    """A NaN ranks below -inf and sets status 1; fewer score columns than
    visible buckets rank the columns present and set status 2."""
    members = np.arange(8 * 4, dtype=np.int32).reshape(8, 4)
    scores = np.array([[0.5, np.nan, -np.inf, 0.5, -0.0, 0.0, 1.0, 2.0]], np.float32)
    lists, lengths, picked, status = oracle_lib.dlsa_select(
        scores, members, np.array([100]), total_rows=8, window=4, sink=0, top_k=100,
        top_p=8, buckets_per_block=1)
    assert list(picked[0]) == [7, 6, 0, 3, 4, 5, 2, 1]
    assert status[0] == 1
    _, _, picked2, status2 = oracle_lib.dlsa_select(
        scores[:, :3], members, np.array([100]), total_rows=8, window=4, sink=0, top_k=4,
        top_p=2, buckets_per_block=1)
    assert status2[0] == 3 and list(picked2[0]) == [0, 2]
