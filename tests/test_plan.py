"""The matmul launch plan on the host (snk_q4_plan, no GPU): a plan depends on (N, K, weight type) alone, and its
k-slices stay within what the row kernels after a layer matrix add (KS_MAX = 16), also for matrices deeper than
Qwen3-4B's: the down projections of Qwen3-14B (5120 x 17408) and Qwen3-32B (5120 x 25600) take longer slices."""
import pytest

import sllm_next as S

KS_MAX = 16


@pytest.mark.parametrize("wt", [2, 8])
@pytest.mark.parametrize("N,K", [(5120, 17408), (5120, 25600), (4096, 27648), (2560, 9728), (2560, 4096),
                                 (19456, 2560), (6144, 2560), (256, 17408), (256, 25600), (2048, 6144)])
def test_plan_slices_within_bound(N, K, wt):
    spw, ks = S.q4_plan(N, K, wt)
    ngroups = (K // 32 + 3) // 4
    assert 1 <= ks <= KS_MAX, (N, K, wt, ks)
    # whole slices of an even number of groups: ks slices of gps groups cover the groups, the last one not empty
    gps = -(-ngroups // ks)
    gps += gps % 2
    assert (ks - 1) * gps < ngroups <= ks * gps, (N, K, ks, gps)


def test_plan_of_known_shapes():
    # Qwen3-4B's matrices keep their slices (the streaming kernel's plans); the deep ones grow theirs
    assert S.q4_plan(2560, 9728) == (1, 10)
    assert S.q4_plan(19456, 2560) == (1, 3)
    assert S.q4_plan(5120, 17408) == (1, 14)  # 10 groups a slice
    assert S.q4_plan(5120, 25600) == (1, 15)  # 14 groups a slice
