"""The RoPE / QK-norm oracle pinned by closed forms (no retyping of its formulas)."""

import math

import numpy as np
import torch

from oracle.rope import (permute_for_rope, qk_norm_rope, rms_norm, rope_frequencies, rope_interleaved,
                         token_positions)


def test_permute_index_definition():
    x = torch.arange(2 * 3 * 8, dtype=torch.float32).view(2, 3, 8)
    y = permute_for_rope(x)
    for i in range(4):
        assert torch.equal(y[..., 2 * i], x[..., i]) and torch.equal(y[..., 2 * i + 1], x[..., 4 + i])


def test_rms_norm_of_constant_vector_is_the_weight():
    w = (torch.randn(128) * 0.5 + 1).to(torch.bfloat16)
    x = torch.full((3, 4, 128), 2.0, dtype=torch.bfloat16)
    assert torch.equal(rms_norm(x, w, 1e-6), w.expand(3, 4, 128))  # 2 * rsqrt(4 + 1e-6) rounds to 1.0
    x = torch.full((1, 1, 128), -0.25, dtype=torch.bfloat16)
    assert torch.equal(rms_norm(x, w, 1e-6)[0, 0], -w)


def test_rope_closed_forms():
    g = torch.Generator().manual_seed(0)
    f = rope_frequencies(128, 1e6)
    assert f[0] == 1.0 and abs(float(f[-1]) - 1e6 ** (-126 / 128)) < 1e-12
    x = torch.randn(3, 2, 128, generator=g, dtype=torch.float64)
    # position 0: the identity
    assert torch.equal(rope_interleaved(x, np.zeros(3, np.int64), f), x)
    # every pair keeps its length
    y = rope_interleaved(x, np.array([1, 777, 31000]), f)
    nx = x[..., 0::2] ** 2 + x[..., 1::2] ** 2
    ny = y[..., 0::2] ** 2 + y[..., 1::2] ** 2
    assert torch.allclose(nx, ny, rtol=1e-12)
    # counter-clockwise turn of each pair as a complex number: (a + ib) e^{i p f}
    p = 777
    ang = (np.float32(p) * f).astype(np.float32).astype(np.float64)
    z = torch.complex(x[1, :, 0::2], x[1, :, 1::2]) * torch.exp(1j * torch.from_numpy(ang))
    assert torch.allclose(y[1, :, 0::2], z.real) and torch.allclose(y[1, :, 1::2], z.imag)
    # q.k depends only on the position difference
    q, k = x[:1], x[1:2]
    def dot(m, n):
        return float((rope_interleaved(q, np.array([m]), f) * rope_interleaved(k, np.array([n]), f)).sum())
    assert abs(dot(10, 3) - dot(110, 103)) < 1e-3 * abs(dot(10, 3)) + 1e-6
    assert abs(dot(500, 0) - dot(1500, 1000)) < 1e-3 * abs(dot(500, 0)) + 1e-6


def test_llama31_frequency_regions():
    cfg = dict(low_freq_factor=1.0, high_freq_factor=4.0, old_context_len=8192.0)
    scale = 8.0
    base = rope_frequencies(128, 500000.0)
    f = rope_frequencies(128, 500000.0, scale, cfg)
    wl = 2 * math.pi / base.astype(np.float64)
    high = wl < 8192 / 4.0
    low = wl > 8192 / 1.0
    mid = ~high & ~low
    assert high.any() and low.any() and mid.any()
    assert np.array_equal(f[high], base[high])                        # short wavelengths: unchanged
    assert np.allclose(f[low], base[low] / scale, rtol=1e-6)           # long wavelengths: divided by the scale
    # the interpolated band lies between its two limits
    assert np.all((f[mid] <= base[mid] * (1 + 1e-6)) & (f[mid] >= base[mid] / scale * (1 - 1e-6)))


def test_positions_from_rows():
    pos = token_positions([0, 3, 3, 5, 8], [100, 7, 50, 0], 9)
    assert pos.tolist() == [100, 101, 102, 50, 51, 0, 1, 2, -1]


def test_composed_sequence_matches_stepwise():
    g = torch.Generator().manual_seed(1)
    q = torch.randn(5, 4, 128, generator=g).to(torch.bfloat16)
    k = torch.randn(5, 2, 128, generator=g).to(torch.bfloat16)
    wq = (torch.rand(128, generator=g) + 0.5).to(torch.bfloat16)
    wk = (torch.rand(128, generator=g) + 0.5).to(torch.bfloat16)
    qo, ko = qk_norm_rope(q, k, [0, 2, 5], [40, 9], theta=1e6, q_weight=wq, k_weight=wk)
    f = rope_frequencies(128, 1e6)
    pos = np.array([40, 41, 9, 10, 11])
    assert torch.equal(qo, rope_interleaved(permute_for_rope(rms_norm(q, wq, 1e-6)), pos, f))
    assert torch.equal(ko, rope_interleaved(permute_for_rope(rms_norm(k, wk, 1e-6)), pos, f))


def test_native_frequency_table_equals_oracle():
    """aspire_rope_frequencies (host code of the HIP library) against the restatement."""
    from aspire_amd.attention.rope import RopeConfig, rope_frequencies as native
    for cfg, ll in ((RopeConfig(1e6), None), (RopeConfig(10000.0, 2.0), None),
                    (RopeConfig(500000.0, 8.0, 1.0, 4.0, 8192),
                     dict(low_freq_factor=1.0, high_freq_factor=4.0, old_context_len=8192.0))):
        assert np.array_equal(native(128, cfg).numpy(), rope_frequencies(128, cfg.rope_theta, cfg.rope_scale, ll))
