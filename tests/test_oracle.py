"""Pins the CPU oracle against known answers that do not restate its formulas.

* the reference's own closed-form long-context test (tests/test_cuda.py:237-273)
* IEEE binary16 bit patterns, sigmoid values, RMSNorm of a constant row
* RoPE on one-hot rows with non-uniform gamma (fixes the pair (i, i+32), the
  sign of the rotation, the base 1e7 and the order RMS -> gamma -> RoPE)
* torch's scaled_dot_product_attention in float64 for the raw GQA core
* invariants: single key, equal keys, causality, grouped == sequential
* input/output vectors of the reference's own CPU attention on its sine-wave
  fixture (tests/golden/fused_attention.npz, written by the script beside it)
"""
import math
from pathlib import Path

import numpy as np
import pytest
import torch

from oracle import attention_ref as ref
from oracle import kat
from redshift_amd.workloads import WORKLOADS, make_inputs, to_float


def test_half_matches_binary16_bit_patterns():
    for value, bits in kat.HALF_BITS:
        with np.errstate(over='ignore'):
            got = np.float16(ref.half(value)).view(np.uint16)
        assert int(got) == bits, (value, hex(int(got)), hex(bits))


def test_sigmoid_known_values():
    assert ref.sigmoid(0.0) == 0.5
    assert abs(ref.sigmoid(math.log(3.0)) - 0.75) < 1e-15
    assert abs(ref.sigmoid(-math.log(3.0)) - 0.25) < 1e-15


def test_rmsnorm_of_constant_row():
    gamma = 1 + np.arange(256) / 512
    for c in (0.0, 0.3, -2.5):
        got = ref.rmsnorm(np.full(256, c), gamma, 1e-6)
        want = c / math.sqrt(c * c + 1e-6) * gamma
        np.testing.assert_allclose(got, want, rtol=1e-14, atol=1e-300)


@pytest.mark.parametrize('i', [0, 1, 17, 31, 32, 45, 63])
@pytest.mark.parametrize('pos', [0, 1, 7, 2047, 139263])
def test_prepare_one_hot_closed_form(i, pos):
    gamma = 1 - np.arange(256) / 512          # non-uniform: pins RMS -> gamma -> RoPE
    row = np.zeros(256)
    row[i] = 0.7
    got = ref.prepare(row, gamma, pos, 1e-6)
    want = kat.rope_one_hot(i, pos, gamma, 1e-6, amplitude=0.7)
    np.testing.assert_allclose(got, want, rtol=0, atol=1e-12)


def test_rope_leaves_dims_64_and_up():
    rng = np.random.default_rng(5)
    row = rng.standard_normal(256)
    out = ref.rope(row, 1234)
    np.testing.assert_array_equal(out[64:], row[64:])
    # a rotation keeps the norm of every pair
    np.testing.assert_allclose(out[:32] ** 2 + out[32:64] ** 2, row[:32] ** 2 + row[32:64] ** 2, rtol=1e-12)


@pytest.mark.parametrize('position,batch', [(2047, 3), (32767, 1), (139263, 1)])
def test_fused_attention_long_context_closed_form(position, batch):
    c = kat.long_context_case(position, batch)
    out, kc, vc = ref.fused_attention(c['key_cache'], c['value_cache'], c['q_gate'], c['key'],
                                      c['value'], c['q_norm'], c['k_norm'], batch, position,
                                      c['epsilon'])
    e = c['expected'].reshape(-1)
    assert np.max(np.abs(out - e) / (1 + np.abs(e))) < 1e-12
    n = position * 1024
    np.testing.assert_array_equal(kc[:n], c['key_cache'].reshape(-1).astype(np.float64))
    np.testing.assert_array_equal(vc[:n], c['value_cache'].reshape(-1).astype(np.float64))
    np.testing.assert_array_equal(kc[n:], 0.0)
    np.testing.assert_array_equal(vc[n:], ref.half(c['value']).reshape(-1))


def test_fused_attention_grouped_equals_sequential():
    c = kat.sine_wave_case()
    b, pos = c['batch'], c['position']
    out, kc, vc = ref.fused_attention(c['key_cache'], c['value_cache'], c['q_gate'], c['key'],
                                      c['value'], c['q_norm'], c['k_norm'], b, pos, c['epsilon'])
    seq_k, seq_v = c['key_cache'].reshape(-1), c['value_cache'].reshape(-1)
    rows = []
    for t in range(b):
        o, seq_k, seq_v = ref.fused_attention(seq_k, seq_v, c['q_gate'][t:t + 1], c['key'][t:t + 1],
                                              c['value'][t:t + 1], c['q_norm'], c['k_norm'], 1,
                                              pos + t, c['epsilon'])
        rows.append(o)
    np.testing.assert_allclose(out, np.concatenate(rows), rtol=0, atol=1e-13)
    np.testing.assert_array_equal(kc, seq_k)
    np.testing.assert_array_equal(vc, seq_v)


@pytest.mark.parametrize('batch,position,rows', [(12, 40, [0, 5, 11]), (40, 0, [0, 1, 31, 32, 39]),
                                               (9, 300, list(range(9)))])
def test_fused_attention_rows_equals_fused_attention(batch, position, rows):
    """The selected-rows form (for chunks too long for the per-token loop)
    against the per-token restatement on random inputs: the same rows to
    float64 rounding, the same appended caches bit for bit."""
    rng = np.random.default_rng(batch + position)
    kc = ref.half(rng.standard_normal((position, 4, 256)) * .5)
    vc = ref.half(rng.standard_normal((position, 4, 256)) * .5)
    q_gate = rng.standard_normal((batch, 24, 512))
    key = rng.standard_normal((batch, 4, 256))
    value = rng.standard_normal((batch, 4, 256))
    q_norm = 1 + .25 * rng.uniform(-1, 1, 256)
    k_norm = 1 + .25 * rng.uniform(-1, 1, 256)
    out, k_all, v_all = ref.fused_attention(kc, vc, q_gate, key, value, q_norm, k_norm, batch, position, 1e-6)
    sel, k_sel, v_sel = ref.fused_attention_rows(kc, vc, q_gate, key, value, q_norm, k_norm, batch, position,
                                                 1e-6, rows)
    np.testing.assert_allclose(sel, out.reshape(batch, 24, 256)[rows], rtol=0, atol=1e-12)
    np.testing.assert_array_equal(k_sel.reshape(-1), k_all)
    np.testing.assert_array_equal(v_sel.reshape(-1), v_all)


def _sdpa_reference(q, k, v, position, scale):
    """torch float64 SDPA with an explicit causal mask and kv heads repeated."""
    T, Hq, D = q.shape
    n = position + T
    G = Hq // k.shape[1]
    qt = torch.from_numpy(np.asarray(q, np.float64)).permute(1, 0, 2)               # [Hq, T, D]
    kt = torch.from_numpy(np.asarray(k[:n], np.float64)).permute(1, 0, 2).repeat_interleave(G, 0)
    vt = torch.from_numpy(np.asarray(v[:n], np.float64)).permute(1, 0, 2).repeat_interleave(G, 0)
    mask = torch.arange(n)[None, :] <= (position + torch.arange(T))[:, None]
    o = torch.nn.functional.scaled_dot_product_attention(qt, kt, vt, attn_mask=mask, scale=scale)
    return o.permute(1, 0, 2).numpy()


@pytest.mark.parametrize('T,Hq,Hkv,D,position', [
    (1, 8, 2, 128, 127), (1, 24, 4, 256, 40), (8, 24, 4, 256, 33), (3, 6, 6, 16, 0),
    (5, 12, 3, 64, 100), (16, 4, 1, 32, 7)])
def test_gqa_core_matches_torch_sdpa(T, Hq, Hkv, D, position):
    rng = np.random.default_rng(T * 1000 + position)
    n = position + T
    q = rng.standard_normal((T, Hq, D))
    k = rng.standard_normal((n, Hkv, D))
    v = rng.standard_normal((n, Hkv, D))
    scale = 1 / math.sqrt(D)
    want = _sdpa_reference(q, k, v, position, scale)
    np.testing.assert_allclose(ref.gqa_attention(q, k, v, position, scale), want, rtol=0, atol=1e-12)
    np.testing.assert_allclose(ref.gqa_attention_fp32(q, k, v, position, scale), want, rtol=0, atol=2e-5)
    rows = [0, T - 1]
    np.testing.assert_allclose(ref.gqa_attention(q, k, v, position, scale, rows=rows), want[rows],
                               rtol=0, atol=1e-12)


def test_gqa_core_invariants():
    rng = np.random.default_rng(11)
    D = 32
    # one visible key: output is that key's value row
    q = rng.standard_normal((1, 4, D))
    k = rng.standard_normal((1, 2, D))
    v = rng.standard_normal((1, 2, D))
    out = ref.gqa_attention(q, k, v, 0, 0.3)
    np.testing.assert_allclose(out[0, :2], np.repeat(v[0, :1], 2, 0), atol=1e-15)
    np.testing.assert_allclose(out[0, 2:], np.repeat(v[0, 1:], 2, 0), atol=1e-15)
    # identical keys: output is the mean of the visible values
    k = np.repeat(rng.standard_normal((1, 2, D)), 9, 0)
    v = rng.standard_normal((9, 2, D))
    out = ref.gqa_attention(q, k, v, 8, 0.3)
    np.testing.assert_allclose(out[0, 0], v[:, 0].mean(0), atol=1e-14)
    # causality: keys past position+t do not change row t
    q = rng.standard_normal((3, 4, D))
    k = rng.standard_normal((12, 2, D))
    v = rng.standard_normal((12, 2, D))
    a = ref.gqa_attention(q, k, v, 9, 0.2)
    k2, v2 = k.copy(), v.copy()
    k2[10:] *= 100
    v2[10:] = np.nan
    b = ref.gqa_attention(q, k2, v2, 9, 0.2)
    np.testing.assert_array_equal(a[0], b[0])


def test_cpu_plumbing_workload_against_sdpa():
    w = WORKLOADS['cpu_plumbing']
    q, k, v, _ = make_inputs(w)
    want = _sdpa_reference(to_float(q, w.dtype), to_float(k, w.dtype), to_float(v, w.dtype), w.position, w.scale)
    np.testing.assert_allclose(ref.gqa_attention(q, k, v, w.position, w.scale), want, atol=1e-12)
    np.testing.assert_allclose(ref.gqa_attention_fp32(q, k, v, w.position, w.scale), want, atol=2e-5)


GOLDEN = Path(__file__).resolve().parent / 'golden' / 'fused_attention.npz'


def golden_cases():
    z = np.load(GOLDEN)
    for batch, position in z['cases']:
        tag = f'b{batch}_p{position}'
        yield int(batch), int(position), {k[len(tag) + 1:]: z[k] for k in z.files if k.startswith(tag + '_')}


@pytest.mark.parametrize('case', list(golden_cases()), ids=lambda c: f'b{c[0]}_p{c[1]}')
def test_fused_attention_matches_reference_vectors(case):
    """The oracle against the reference's own tests/cpu_reference.py output
    on its sine-wave fixture (RoPE on q and k at positions 5..47, norm
    weights 1 +- i/512, gate): output to the float32 storage of the vectors,
    appended K/V rows bit for bit."""
    batch, position, g = case
    out, kc, vc = ref.fused_attention(g['kc'][:position].astype(np.float64), g['vc'][:position].astype(np.float64),
                                      g['q_gate'], g['key'], g['value'], g['q_norm'], g['k_norm'],
                                      batch, position, 1e-6)
    e = g['out'].astype(np.float64).reshape(-1)
    assert np.max(np.abs(out - e) / (1 + np.abs(e))) < 1e-7   # the float32 storage's own rounding
    np.testing.assert_array_equal(np.asarray(kc, np.float64), g['kc'].astype(np.float64).reshape(-1))
    np.testing.assert_array_equal(np.asarray(vc, np.float64), g['vc'].astype(np.float64).reshape(-1))
