"""Training integration on the CPU: codebooks, Newton-Schulz, the GPT's
construction, initialisation, optimizer split, rotary embedding and the
soft-capped loss (closed forms and autograd of the plain expression)."""
from __future__ import annotations

import math

import pytest
import torch

from losslessly_compressed_tensors_amd.comp_format import DistType, NoiseLevel


def test_default_codebooks():
    """LCT/components/dist_configs.py:4-35 and examples/nanogpt/dist_configs.py:4-7."""
    from losslessly_compressed_tensors_amd.components import dist_configs as d
    expected = {
        "weight_dist": (DistType.LAPLACE, NoiseLevel.CLEAN, 0.0),
        "momentum_dist": (DistType.EMPIRICAL, NoiseLevel.CLEAN, 0.02),
        "momentum_first_dist": (DistType.EMPIRICAL, NoiseLevel.CLEAN, 0.5),
        "act_dist": (DistType.LAPLACE, NoiseLevel.CLEAN, 0.0),
        "act_relu_dist": (DistType.LAPLACE, NoiseLevel.CLEAN, 0.5),
    }
    for name, (family, noise, zero_prob) in expected.items():
        dist = getattr(d, name)
        assert (dist.family, dist.noise_level, dist.zero_prob, dist.param, dist.mean) == (
            family, noise, zero_prob, 1.0, 0.0), name
    from examples.nanogpt import train_gpt_lct as gpt
    assert (gpt.weight_dist.family, gpt.weight_dist.zero_prob) == (DistType.LAPLACE, 0.01)
    assert (gpt.act_relu_dist.noise_level, gpt.act_relu_dist.zero_prob) == (NoiseLevel.SPARSE, 0.5)
    assert gpt.momentum_dist.zero_prob == 0.02 and gpt.act_dist.zero_prob == 0.0


@pytest.mark.parametrize("shape", [(64, 128), (128, 64)])
def test_newton_schulz_orthogonalises(shape):
    """12 cubic iterations drive every singular value of a random matrix to
    about 1 (the map s -> 2s - 1.5s^3 + 0.5s^5 has a superattracting fixed
    point at 1), and the result keeps G's shape and orientation."""
    from losslessly_compressed_tensors_amd.components.sparse_utils import (
        zeropower_via_newtonschulz5)
    g = torch.randn(*shape, generator=torch.Generator().manual_seed(0))
    x = zeropower_via_newtonschulz5(g, 12)
    assert x.shape == g.shape and x.dtype == torch.bfloat16
    s = torch.linalg.svdvals(x.float())
    assert s.min() > 0.9 and s.max() < 1.1
    # Same singular vectors: X ~ U V^T of G.
    u, _, vh = torch.linalg.svd(g, full_matrices=False)
    assert torch.allclose(x.float(), u @ vh, atol=0.05)


def test_muon_update_scale_and_state():
    from losslessly_compressed_tensors_amd.components.sparse_utils import muon_update
    g = torch.randn(128, 32, generator=torch.Generator().manual_seed(1)).bfloat16()
    m = torch.zeros_like(g)
    update = muon_update(g.clone(), m, mu=0.95, ns_iters=12)
    # lerp toward g with weight 0.05 from zero: m = 0.05 g (one BF16 rounding).
    assert torch.equal(m, torch.lerp(torch.zeros_like(g), g, 0.05))
    s = torch.linalg.svdvals(update.float())
    assert abs(float(s.mean()) - math.sqrt(128 / 32)) < 0.1 * math.sqrt(128 / 32)


def _tiny_model():
    from examples.nanogpt import train_gpt_lct as gpt
    torch.manual_seed(0)
    model = gpt.GPT(vocab_size=512, num_layers=2, model_dim=128, head_dim=64)
    gpt.initialize_model(model)
    return gpt, model


def test_gpt_structure_and_initialisation():
    gpt, model = _tiny_model()
    names = dict(model.named_parameters())
    assert names["embed.weight"].dtype == torch.bfloat16
    assert names["blocks.0.attn.q.weight"].dtype == torch.bfloat16
    assert names["blocks.0.attn.q.bias"].dtype == torch.float32
    assert model.blocks[0].attn.num_heads == 2
    for name, p in names.items():
        if name.endswith("bias"):
            assert not p.any(), name
        elif name.endswith("gains"):
            assert (p == 1).all(), name
        elif "proj" in name:
            assert not p.any(), name
    q = names["blocks.1.mlp.fc.weight"].detach().float()
    assert abs(float(q.std()) - math.sqrt(0.33 / 128)) < 0.1 * math.sqrt(0.33 / 128)
    assert abs(float(names["embed.weight"].detach().float().std()) - 1) < 0.05


def test_optimizer_split():
    gpt, model = _tiny_model()
    adam, muon = gpt.make_optimizers(model, compressed=False)
    named = dict(model.named_trainable_tensors())
    muon_ids = {id(p) for p in muon.params}
    expected = {id(p) for n, p in named.items() if n.startswith("blocks.") and p.ndim >= 2}
    assert muon_ids == expected and len(muon.params) == 2 * 6
    assert [g["lr"] for g in adam.param_groups] == [0.3, 1 / 320, 0.01]
    assert muon.ns_iters == 12 and muon.first_step and muon.lr == 0.035
    assert float(muon.decay) == pytest.approx(1 - 0.035 * 0.025)


def test_random_tokens_deterministic():
    from examples.nanogpt import train_gpt_lct as gpt
    a, t = gpt.random_tokens(2, 16, "cpu", seed=5)
    b, u = gpt.random_tokens(2, 16, "cpu", seed=5)
    assert torch.equal(a, b) and torch.equal(t, u)
    assert a.dtype == torch.int32 and t.dtype == torch.int64
    assert torch.equal(a[:, 1:].long(), t[:, :-1])
    assert int(a.max()) < gpt.TOKEN_IDS and int(a.min()) >= 0


def test_rotary_rotates_first_half_pairs():
    from examples.nanogpt import train_gpt_lct as gpt
    rot = gpt.Rotary(64)
    x = torch.randn(1, 8, 2, 64, generator=torch.Generator().manual_seed(2))
    y = rot(x)
    assert torch.equal(y[:, 0], x[:, 0])  # position 0: angle 0
    # Channels j and j + 32 rotate together; the zero-frequency quarter
    # (j = 16..31) stays put.
    assert torch.allclose(y[..., 16:32], x[..., 16:32]) and torch.allclose(y[..., 48:], x[..., 48:])
    pair = lambda t: t[..., :16].square() + t[..., 32:48].square()
    assert torch.allclose(pair(y), pair(x), atol=1e-5)


@pytest.mark.parametrize("rows", [6, 1100])   # one row group, three (512 rows each)
def test_softcap_cross_entropy_matches_autograd(rows):
    from examples.nanogpt import train_gpt_lct as gpt
    g = torch.Generator().manual_seed(3)
    logits = (torch.randn(rows, 40, generator=g) * 20).bfloat16().requires_grad_()
    targets = torch.randint(0, 40, (rows,), generator=g)
    loss = gpt.SoftcapCrossEntropy.apply(logits, targets)
    loss.backward()
    x = logits.detach().double().requires_grad_()
    capped = 15 * x / torch.sqrt(x * x + 225)
    ref = (torch.logsumexp(capped, -1) - capped.gather(1, targets[:, None]).squeeze(1)).sum()
    ref.backward()
    assert float(loss.detach()) == pytest.approx(float(ref.detach()), rel=1e-5)
    assert torch.allclose(logits.grad.double(), x.grad, atol=1e-2, rtol=1e-2)
