"""The reference's RoPE-scheme contract tests (fade tests/test_rope.py:26-98), run
against fade_amd.rope's host tables: same schemes, same assertions and tolerances."""

import torch

from fade_amd.rope import Llama3, LinearScaled, NoRope, NtkAware, Vanilla, Yarn

THETA, HEAD_DIM, DEVICE = 10000.0, 64, torch.device("cpu")


def test_vanilla_inv_freq_shape_and_monotonic():  # tests/test_rope.py:26-32
    inv = Vanilla(theta=THETA, head_dim=HEAD_DIM).inv_freq(DEVICE)
    assert inv.shape == (HEAD_DIM // 2,)
    assert ((inv[1:] - inv[:-1]) < 0).all()


def test_linear_scaled_stretches_positions():  # tests/test_rope.py:35-45
    v = Vanilla(theta=THETA, head_dim=HEAD_DIM)
    ls = LinearScaled(theta=THETA, head_dim=HEAD_DIM, factor=2.0)
    pos = torch.arange(16)
    cos_v, _ = v.compute_cos_sin(pos, DEVICE)
    cos_ls, _ = ls.compute_cos_sin(pos, DEVICE)
    # [1, 1, S, D]: position axis 2
    assert torch.allclose(cos_v[:, :, :1], cos_ls[:, :, :1], atol=1e-6)
    cos_v1, _ = v.compute_cos_sin(torch.tensor([1]), DEVICE)
    assert torch.allclose(cos_v1, cos_ls[:, :, 2:3], atol=1e-5)


def test_ntk_aware_changes_base_theta():  # tests/test_rope.py:48-53
    ntk = NtkAware(theta=THETA, head_dim=HEAD_DIM, factor=2.0)
    van = Vanilla(theta=THETA * 2.0, head_dim=HEAD_DIM)
    assert torch.allclose(ntk.inv_freq(DEVICE), van.inv_freq(DEVICE))


def test_llama3_inv_freq_three_bands():  # tests/test_rope.py:56-74
    l3 = Llama3(theta=THETA, head_dim=HEAD_DIM, factor=4.0, low_freq_factor=1.0, high_freq_factor=4.0,
                original_max_position_embeddings=8192)
    base = Vanilla(theta=THETA, head_dim=HEAD_DIM).inv_freq(DEVICE)
    inv = l3.inv_freq(DEVICE)
    assert inv.shape == base.shape
    assert torch.allclose(inv[:4], base[:4], atol=1e-6)
    assert torch.allclose(inv[-4:], base[-4:] / 4.0, atol=1e-6)


def test_yarn_inv_freq_shape():  # tests/test_rope.py:77-81
    inv = Yarn(theta=THETA, head_dim=HEAD_DIM, factor=2.0).inv_freq(DEVICE)
    assert inv.shape == (HEAD_DIM // 2,) and torch.isfinite(inv).all()


def test_norope_identity_and_vanilla_is_rope():  # tests/test_rope.py:84-98
    nr = NoRope(theta=THETA, head_dim=HEAD_DIM)
    cos, sin = nr.compute_cos_sin(torch.arange(8), DEVICE)
    assert cos.shape == (1, 1, 8, HEAD_DIM) and sin.shape == (1, 1, 8, HEAD_DIM)
    assert torch.allclose(cos, torch.ones_like(cos)) and torch.allclose(sin, torch.zeros_like(sin))
    assert not nr.is_rope
    assert Vanilla(theta=THETA, head_dim=HEAD_DIM).is_rope
