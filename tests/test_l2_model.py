"""The L2 model of the tile GEMM's operand fetch (l2_model.py) against the FETCH_SIZE
measured for the QKV launch (profiles/gemm_i8_qkv_4096x3072x9216_traffic.json), and
what it says about the tile order: each round re-reads its operands past the L2, because
one round's operands per XCD (4 m-tiles x 8 n-tiles of 256x192: 7.9 MB) do not fit the
XCD's 4 MiB L2."""

import json
import os

import l2_model

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def test_the_model_reproduces_the_measured_fetch():
    with open(os.path.join(ROOT, "profiles", "gemm_i8_qkv_4096x3072x9216_traffic.json")) as f:
        measured = json.load(f)["gemm_i8"]["hbm_read_bytes"]
    model = l2_model.fetch_bytes(4096, 9216, 3072, 256, 192)
    assert abs(model - measured) / measured < 0.01, (model, measured)
    # = 3 rounds x 8 XCDs x (1024 A rows + 1536 W rows) x 3072 bytes: every round's
    # operands once, none kept across rounds
    assert model == 3 * 8 * (4 * 256 + 8 * 192) * 3072


def test_a_round_per_xcd_is_already_the_smallest_working_set():
    # 32 concurrent tiles per XCD as a x b m- and n-tiles: 4 x 8 reads the fewest rows.
    def rows(a, b):
        return a * 256 + b * 192
    assert min((rows(a, 32 // a), a) for a in (1, 2, 4, 8, 16, 32))[1] == 4
    # Running odd rounds through K backwards reuses what the L2 still holds of the
    # previous round: about a tenth less, far from the operands' 40.9 MB.
    back = l2_model.fetch_bytes(4096, 9216, 3072, 256, 192, reverse_odd_rounds=True)
    fwd = l2_model.fetch_bytes(4096, 9216, 3072, 256, 192)
    assert 0.85 < back / fwd < 0.95
