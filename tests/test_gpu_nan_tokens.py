"""Token ids that the GPU feeds on by itself stay inside the token table.

The greedy argmax gives -1 for a row without a finite score (NaN scores never win; kernels.metal:327-356 keeps the
first index of the max, and a row of NaN has none). Three paths feed argmax outputs back as token ids without a host
check: the queued (chained) step (sn_step.inc.h:67-78), the guess head's next draft row (sn_cache.inc.h:300-388) and
the fused draft-verify step's verify rows and forced drafts. A model whose output norm weight is NaN makes every
logit NaN, so all three meet -1: the gathers by token give a zero row for an id outside [0, V) and the forced-draft
write skips it, so the steps run to the end inside their buffers, and the host still refuses -1 as an input token."""

import numpy as np
import pytest

import sllm_next as S
from oracle.gguf import GGUF
from tests import gpu_util as U

TINY = dict(n_layer=2, n_embd=256, n_head=8, n_head_kv=2, n_ff=512, n_vocab=1000, nextn=1)
K = 3


def setup_module(module):
    # the GPU is set up before the library is first loaded, as in the other GPU modules (the file's CPU test runs
    # where there is none)
    if U.torch().cuda.is_available():
        U.torch().cuda.init()


def nan_output_norm(path: str) -> None:
    """Overwrite the F32 output_norm.weight of a model file with NaN."""
    g = GGUF(path)
    ne, t, o = g.tinfo["output_norm.weight"]
    start, n = g.data_offset + o, int(np.prod(ne))
    del g
    assert t == 0 and n == TINY["n_embd"]
    with open(path, "r+b") as f:
        f.seek(start)
        f.write(np.full(n, np.nan, np.float32).tobytes())


@pytest.fixture(scope="module")
def nan_model(tmp_path_factory):
    path = str(tmp_path_factory.mktemp("model") / "nan.gguf")
    S.write_model(path, S.model_cfg(**TINY), seed=5)
    nan_output_norm(path)
    return path


def test_the_model_file_has_a_nan_output_norm(nan_model):
    """(CPU) the fixture's file: the output norm is NaN, the other norms finite."""
    g = GGUF(nan_model)
    assert np.all(np.isnan(g.tensor("output_norm.weight")))
    assert np.all(np.isfinite(g.tensor("blk.0.attn_norm.weight")))


def prefill(eng, rng, lens):
    V = TINY["n_vocab"]
    for s, n in enumerate(lens):
        out = eng.step(rng.integers(0, V, n).astype(np.int32), np.full(n, s, np.int32), np.arange(n, dtype=np.int32),
                       np.array([n - 1], np.int32), n_write=0)
        assert out[0] == -1  # every logit is NaN


@pytest.mark.gpu
def test_queued_step_fed_minus_one(nan_model):
    """A chained decode step queues its successor on the GPU with its own tokens, all -1 here."""
    V = TINY["n_vocab"]
    rng = np.random.default_rng(3)
    lens = [9, 14]
    seq = np.arange(2, dtype=np.int32)
    rows = np.arange(2, dtype=np.int32)
    with S.Engine(nan_model, slots=2, ctx=64, max_rows=64) as eng:
        prefill(eng, rng, lens)
        pos = np.array(lens, np.int32)
        for it in range(2):  # the first queues a step fed -1; so does the second, after the first was dropped
            out = eng.step(rng.integers(0, V, 2).astype(np.int32), seq, pos, rows, chain=1)
            assert np.all(out == -1)
            with pytest.raises(S.SnError):  # the host refuses -1 as an input token
                eng.step(out, seq, pos + 1, rows)
            pos = pos + 1
        out = eng.step(rng.integers(0, V, 2).astype(np.int32), seq, pos, rows)
        assert np.all(out == -1)
        assert eng.chain_count() == (0, 2)


@pytest.mark.gpu
def test_guess_head_and_fused_steps_fed_minus_one(nan_model):
    """The guess head's draft rows after the first take the previous draft (-1) from device memory; a fused
    draft-verify step makes verify rows and forced drafts of such drafts."""
    V = TINY["n_vocab"]
    rng = np.random.default_rng(4)
    lens = [9, 14]
    seq = np.arange(2, dtype=np.int32)
    with S.Engine(nan_model, slots=2, ctx=64, max_rows=64) as eng:
        eng.guess_on(True)
        assert eng.guess_head()
        prefill(eng, rng, lens)
        pos = np.array(lens, np.int32)
        g = eng.guess(0, int(rng.integers(0, V)), int(pos[0]), K)
        assert np.all(g == -1)
        last = rng.integers(0, V, 2).astype(np.int32)
        for force in (None, np.ones((2, K), np.uint8)):
            n, t = eng.spec_step(seq, last, pos, K, force=force)
            assert np.all(t == -1) and np.all((n >= 1) & (n <= K + 1))  # (drafts -1 match argmax -1)
            pos = pos + n
        assert np.all(pos < 64)
