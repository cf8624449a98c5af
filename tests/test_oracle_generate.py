"""Pin of the oracle's denoising loop (orc_generate, restating diffuse_sample of
src/diffuse-sampler.cpp:60-370 with the step cache of src/diffuse-cache.h:79-146).

What fixes the loop without re-running it: the unmask counts per step are the
schedule's integer sequences (random-init logits have entropy near ln V, far above
tau = 1.5, so entropy_exit reduces to the schedule), and the rows of each forward
follow from the counts alone:
  * a full step (step 0, cache off, refresh) runs N = P + B rows;
  * a cached step s runs the positions still masked, plus those unmasked at step
    s-1 (their token changed since the last forward), plus, with keep_active = k,
    those unmasked at step s-1-j (j = 1..k) provided step s-j was itself a cached
    step: only a cached step records when a position changed
    (src/diffuse-cache.h:95-105, called only on the cached path,
    src/diffuse-sampler.cpp:158-162).
The cosine sequences below are the ones derived from the schedule formula
(src/diffuse-sampler.cpp:12-31) for B = 256 and 64; linear unmasks B/16 per step.
"""
import numpy as np
import pytest

import dfx
import oracle_py as O
from conftest import TINY_LLADA

COSINE_256 = [1, 4, 6, 8, 11, 13, 15, 17, 19, 20, 22, 23, 23, 24, 25, 25]
COSINE_64 = [1, 1, 2, 2, 3, 3, 4, 4, 5, 5, 5, 5, 6, 6, 6, 6]


def expected_rows(P, B, unmasked, use_cache, refresh=0, keep=0):
    N = P + B
    rows, full = [], []
    masked = B
    for s, u in enumerate(unmasked):
        is_full = not use_cache or s == 0 or (refresh > 0 and s % refresh == 0)
        if is_full:
            r = N
        else:
            r = masked + unmasked[s - 1]
            for j in range(1, keep + 1):
                if s - 1 - j >= 0 and not full[s - j]:
                    r += unmasked[s - 1 - j]
            if r >= N or r == 0:
                r, is_full = N, True
        rows.append(r)
        full.append(is_full)
        masked -= u
    return rows


@pytest.fixture(scope="module")
def llada_q4(tmp_path_factory):
    p = tmp_path_factory.mktemp("gen") / "llada-q4.gguf"
    dfx.synth_model(p, TINY_LLADA, scheme="q4_k_m", seed=11, sigma=0.05, n_threads=4)
    return O.OracleModel(str(p))


@pytest.mark.parametrize("B,sched,counts", [(256, dfx.SCHED_COSINE, COSINE_256), (64, dfx.SCHED_COSINE, COSINE_64),
                                            (256, dfx.SCHED_LINEAR, [16] * 16)])
@pytest.mark.parametrize("remasking,use_cache,refresh,keep", [
    (dfx.ENTROPY_EXIT, True, 0, 0),       # the benchmark's loop
    (dfx.LOW_CONFIDENCE, False, 0, 0),    # no cache: every step full
    (dfx.LOW_CONFIDENCE, True, 5, 0),     # refresh every 5 steps
    (dfx.TOPK_MARGIN, True, 0, 2),        # keep changed positions active 2 more steps
    (dfx.RANDOM, True, 4, 1),
])
def test_orc_generate_rows_and_counts(llada_q4, B, sched, counts, remasking, use_cache, refresh, keep):
    P = 32
    prompt = np.random.default_rng(1).integers(0, 1400, P).astype(np.int32)
    out, st = llada_q4.generate(prompt, B, n_steps=16, schedule=sched, remasking=remasking, use_cache=use_cache,
                                cache_refresh=refresh, cache_keep_active=keep, n_threads=8)
    assert st.actual_steps == 16
    got_counts = list(st.unmasked_per_step[:16])
    assert got_counts == counts
    assert list(st.rows_per_step[:16]) == expected_rows(P, B, counts, use_cache, refresh, keep)
    assert not (out == llada_q4.m.mask_token_id).any()


def test_expected_rows_matches_the_survey_sequence():
    """The benchmark workload's rows per step (32 + 256, cosine, cache on), derived
    independently from the schedule in the workload description."""
    assert expected_rows(32, 256, COSINE_256, True) == [288, 256, 255, 251, 245, 237, 226, 213, 198, 181, 162, 142,
                                                        120, 97, 74, 50]


def test_orc_generate_greedy_tokens_are_row_argmaxes(llada_q4):
    """One step with all positions unmasked at once (n_steps = 1): every generated token
    is the argmax of its own row of one full forward (src/diffuse-sampler.cpp:241-252)."""
    P, B = 16, 24
    prompt = np.random.default_rng(2).integers(0, 1400, P).astype(np.int32)
    out, st = llada_q4.generate(prompt, B, n_steps=1, remasking=dfx.LOW_CONFIDENCE, use_cache=False, n_threads=8)
    seq = np.concatenate([prompt, np.full(B, llada_q4.m.mask_token_id, np.int32)])
    logits = llada_q4.forward_full(seq)
    assert np.array_equal(out, logits[P:].argmax(1))
