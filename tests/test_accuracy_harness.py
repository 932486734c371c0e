"""CPU checks of the teacher-forcing harness (tests/accuracy.py): the oracle against its own
reference run scores perfectly, and a model with a planted mistake is caught."""
import numpy as np

from oracle.model import OracleModel
from tests.accuracy import log_softmax, reference_run, teacher_forcing
from tests.model_weights import random_weights

CFG = dict(n_layer=1, n_embd=256, n_head=4, n_head_kv=2, head_dim=64, n_ff=512, n_vocab=512, norm_eps=1e-5,
           rope_theta=500000.0, rope_neox=0, qk_norm=0, max_ctx=64, max_batch=16)


def test_log_softmax_closed_form():
    z = np.array([0.0, np.log(3.0)])
    assert np.allclose(log_softmax(z), [np.log(0.25), np.log(0.75)])


class Planted:
    """The oracle, except that from the `bad`-th call on the top token's logit is pushed below the
    runner-up (a wrong argmax and a large log-prob error at those positions)."""

    def __init__(self, oracle, bad):
        self.o, self.calls, self.bad = oracle, 0, bad

    def forward(self, tokens):
        lg = np.array(self.o.forward(tokens), np.float64)
        self.calls += 1
        if self.calls > self.bad:
            i = int(np.argmax(lg))
            lg[i] = np.sort(lg)[-2] - 1.0
        return lg


def test_teacher_forcing_scores():
    w = random_weights(CFG, 3)
    prompt = np.array([5, 17, 99, 3], np.int32)
    ref = reference_run(OracleModel(CFG, w), prompt, 6)
    assert len(ref) == 6 and all(len(g["top"]) == 5 for g in ref)
    r = teacher_forcing(OracleModel(CFG, w), prompt, ref)
    assert r["agree"] == 6 and r["max_abs_dlogp"] == 0.0 and r["top5_overlap"] == 1.0
    # 4 prompt calls + 5 forced calls; the last 3 compared positions go wrong
    r = teacher_forcing(Planted(OracleModel(CFG, w), bad=6), prompt, ref)
    assert r["agree"] == 3 and r["max_abs_dlogp"] > 0.5
