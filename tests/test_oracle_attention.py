"""Pins the attention oracle (CPU only): library routine, identities, fp64 form.

Each check is chosen so that a plausible slip in the oracle (a dropped bias, a
wrong scale, a transposed operand, a missing P rounding) fails at least one of
them; `test_checks_have_teeth` plants such slips and asserts they are caught.
"""
from __future__ import annotations

import math

import pytest
import torch

from oracle import attention as oracle
from tests._tol import rel_error


def _inputs(seed, b=1, h=2, nq=37, nk=29, d=64, dtype=torch.float32, mass_max=8):
    g = torch.Generator().manual_seed(seed)
    q = torch.randn(b, h, nq, d, generator=g).to(dtype)
    k = torch.randn(b, h, nk, d, generator=g).to(dtype)
    v = torch.randn(b, h, nk, d, generator=g).to(dtype)
    mass = torch.randint(1, mass_max + 1, (nk,), generator=g).float()
    return q, k, v, mass


def test_matches_sdpa_with_float_mask():
    q, k, v, mass = _inputs(0)
    out = oracle.mass_bias_attention(q, k, v, mass.log())
    ref = oracle.sdpa_with_log_mass(q, k, v, mass.log())
    assert rel_error(out, ref) < 1e-5


def test_unit_mass_is_plain_sdpa():
    q, k, v, _ = _inputs(1)
    out = oracle.mass_bias_attention(q, k, v, torch.zeros(k.shape[-2]))
    ref = torch.nn.functional.scaled_dot_product_attention(q, k, v)
    assert rel_error(out, ref) < 1e-5
    assert rel_error(oracle.mass_bias_attention(q, k, v, None), ref) < 1e-5


def test_key_duplication_identity():
    # Integer mass m_j == key/value j repeated m_j times in plain softmax attention.
    q, k, v, mass = _inputs(2, nk=23)
    reps = mass.long()
    k_dup = torch.repeat_interleave(k, reps, dim=2)
    v_dup = torch.repeat_interleave(v, reps, dim=2)
    dup = torch.nn.functional.scaled_dot_product_attention(q.double(), k_dup.double(), v_dup.double())
    out = oracle.mass_bias_attention(q.double(), k.double(), v.double(), mass.double().log())
    assert rel_error(out, dup) < 1e-10


def test_bias_shift_and_key_permutation_invariance():
    q, k, v, mass = _inputs(3)
    base = oracle.mass_bias_attention(q.double(), k.double(), v.double(), mass.double().log())
    shifted = oracle.mass_bias_attention(q.double(), k.double(), v.double(), mass.double().log() + 3.25)
    assert rel_error(shifted, base) < 1e-12
    perm = torch.randperm(k.shape[-2], generator=torch.Generator().manual_seed(9))
    permuted = oracle.mass_bias_attention(q.double(), k.double()[:, :, perm], v.double()[:, :, perm],
                                          mass.double().log()[perm])
    assert rel_error(permuted, base) < 1e-12


def test_brute_force_loops_tiny():
    q, k, v, mass = _inputs(4, b=1, h=1, nq=3, nk=5, d=64)
    out = oracle.mass_bias_attention(q.double(), k.double(), v.double(), mass.double().log())
    for i in range(3):
        logits = [float(q[0, 0, i].double() @ k[0, 0, j].double()) / 8.0 + math.log(float(mass[j]))
                  for j in range(5)]
        top = max(logits)
        w = [math.exp(x - top) for x in logits]
        row = sum(w[j] * v[0, 0, j].double() for j in range(5)) / sum(w)
        assert rel_error(out[0, 0, i], row) < 1e-12


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_low_precision_rounds_bias_and_probabilities(dtype):
    q, k, v, mass = _inputs(5, dtype=dtype, nk=300)
    out = oracle.mass_bias_attention(q, k, v, mass.log())
    exact = oracle.mass_bias_attention(q.double(), k.double(), v.double(),
                                       mass.log().to(dtype).double())
    assert out.dtype == dtype
    assert rel_error(out, exact) < 2e-2


def test_checks_have_teeth():
    q, k, v, mass = _inputs(6)
    ref = oracle.sdpa_with_log_mass(q, k, v, mass.log())
    dropped_bias = oracle.mass_bias_attention(q, k, v, None)
    wrong_scale = oracle.mass_bias_attention(q * 2, k, v, mass.log())
    transposed = oracle.mass_bias_attention(q, v, k, mass.log())
    negated_bias = oracle.mass_bias_attention(q, k, v, -mass.log())
    for bad in (dropped_bias, wrong_scale, transposed, negated_bias):
        assert rel_error(bad, ref) > 1e-2
