"""The rule that decides when sn_step replays a captured HIP graph, checked on the host (no GPU): the key of a step
holds every host value its launches take, so two steps share a graph only when they would launch the same kernels
with the same arguments. The reference has no graphs; what the key protects is its step semantics (a step computes
what its rows ask, sn_step.inc.h:145-185)."""
import numpy as np
import pytest

import sllm_next as S

# The attention plan's fields in the key: form, items, merge rows, the offsets of groups, items and merge rows, run
# items and their offset, then the fold's: plain chunk items, groups, the most chunks of a group
ATTN_FIELDS = 11


def rows(n, pos):
    return np.arange(n, dtype=np.int32), np.full(n, pos, np.int32)


@pytest.mark.parametrize("page_cells,long_pos", [(64, 3000), (32, 1400)])
def test_chunk_and_whole_forms_have_different_keys(page_cells, long_pos):
    """32 decode rows whose contexts fit one 256-cell chunk (per-chunk items: 32 items and a merge of 32 rows) against
    32 rows with long alike contexts (whole groups on 32 x 8 = 256 workgroups: 32 items, no merge). Everything else a
    launch takes is the same, so the attention form alone must tell the keys apart."""
    k_chunk, w_chunk = S.step_key(32, 8, page_cells, -1, *rows(32, 100))
    k_whole, w_whole = S.step_key(32, 8, page_cells, -1, *rows(32, long_pos))
    assert not w_chunk and w_whole
    assert len(k_chunk) == len(k_whole)
    # the same in every field but the attention list's (so the case is the colliding one) ...
    assert k_chunk[:-ATTN_FIELDS] == k_whole[:-ATTN_FIELDS]
    a_chunk, a_whole = k_chunk[-ATTN_FIELDS:], k_whole[-ATTN_FIELDS:]
    # (form, items, merge rows, groups' offset, items' offset, merge rows' offset): the item count and the offsets of
    # the groups and items agree, which alone left the two forms on one graph
    assert a_chunk[1] == a_whole[1] == 32 and a_chunk[3:5] == a_whole[3:5]
    assert (a_chunk[0], a_chunk[2]) == (0, 32) and (a_whole[0], a_whole[2]) == (1, 0)
    assert a_chunk[6] == a_whole[6] == 0  # no run items (decode rows)
    # ... and the keys differ
    assert k_chunk != k_whole


def test_forced_forms_differ_and_positions_do_not_matter():
    seq, pos = rows(32, 3000)
    k0, w0 = S.step_key(32, 8, 64, 0, seq, pos)
    k1, w1 = S.step_key(32, 8, 64, 1, seq, pos)
    assert (w0, w1) == (False, True) and k0 != k1
    # positions are staged data: a step one cell on (same chunk count) replays the same graph
    assert S.step_key(32, 8, 64, -1, seq, pos + 1)[0] == S.step_key(32, 8, 64, -1, seq, pos)[0]
    # one more chunk changes the item count, so the key
    assert S.step_key(32, 8, 64, 0, seq, pos + 256)[0] != k0


def test_group_shapes_change_the_key():
    """Verify rows (4 consecutive positions of one sequence form one query group at G = 4) against the same number of
    decode rows of distinct sequences: other groups, items and merge rows."""
    seq = np.repeat(np.arange(8, dtype=np.int32), 4)
    pos = np.tile(np.arange(4, dtype=np.int32), 8) + 50
    kv, _ = S.step_key(32, 8, 64, -1, seq, pos)
    kd, _ = S.step_key(32, 8, 64, -1, *rows(32, 50))
    assert kv != kd


def test_bad_arguments_are_refused():
    with pytest.raises(S.SnError):
        S.step_key(32, 7, 64, -1, *rows(4, 10))  # G not a divisor of 16
    with pytest.raises(S.SnError):
        S.step_key(32, 8, 48, -1, *rows(4, 10))  # page size


def test_prompt_run_items_change_the_key():
    """512 prompt rows of one sequence: the planner's run items (128 groups of 4 rows in 32 items, 256 workgroups)
    against the same rows forced to per-chunk items (mode 0): the run-item count is in the key."""
    seq = np.zeros(512, np.int32)
    pos = np.arange(1536, 2048, dtype=np.int32)
    k_run, _ = S.step_key(32, 8, 64, -1, seq, pos)
    k_chunk, _ = S.step_key(32, 8, 64, 0, seq, pos)
    assert k_run[-ATTN_FIELDS:][6] == 32 and k_chunk[-ATTN_FIELDS:][6] == 0
    assert k_run != k_chunk
    # 64 prompt rows make 4 run items, 32 workgroups: too few, the planner keeps chunk items; mode 2 takes them
    assert S.step_key(32, 8, 64, -1, seq[:64], pos[:64])[0][-ATTN_FIELDS:][6] == 0
    assert S.step_key(32, 8, 64, 2, seq[:64], pos[:64])[0][-ATTN_FIELDS:][6] == 4
