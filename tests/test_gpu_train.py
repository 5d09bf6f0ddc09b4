"""Training integration on the GPU: layers, optimizers and a small GPT.

The codec is lossless, so the pinning property of every compressed layer is
bit-identity with the same layer run without compression (outputs and every
gradient), and the layers' compressed branch is checked to have run.  The
optimizers' fused updates are checked element by element against the oracle's
pointwise arithmetic (``oracle.apply_array``: FP32 fused multiply-add, one
round-to-nearest-even to BF16), and their decode/encode round trips against
the same optimizer kept dense.
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

import oracle
from tests.gpu_util import bits_of, require_gpu

pytestmark = pytest.mark.gpu

DEV = "cuda:0"


def _bf16(*shape, seed, scale=1.0):
    g = torch.Generator().manual_seed(seed)
    return (torch.randn(*shape, generator=g) * scale).to(torch.bfloat16).to(DEV)


def _f32(*shape, seed, scale=1.0):
    g = torch.Generator().manual_seed(seed)
    return (torch.randn(*shape, generator=g) * scale).to(DEV)


@pytest.fixture()
def layers_counting(monkeypatch):
    """The layers module with the tensors it compresses counted (one
    ``compress`` each, or one ``compress_batch`` for the queued ones)."""
    from losslessly_compressed_tensors_amd.components import layers
    calls = []
    real, real_batch = layers.compress, layers.compress_batch

    def counting(x, *args, **kwargs):
        calls.append(tuple(x.shape))
        return real(x, *args, **kwargs)

    def counting_batch(xs, *args, **kwargs):
        calls.extend(tuple(x.shape) for x in xs)
        return real_batch(xs, *args, **kwargs)

    monkeypatch.setattr(layers, "compress", counting)
    monkeypatch.setattr(layers, "compress_batch", counting_batch)
    return layers, calls


def _buffer(mib=32):
    from losslessly_compressed_tensors_amd.tensor_buffer import TensorBuffer
    return TensorBuffer(mib * 2 ** 20, device=DEV)


def _run(fn, inputs, grad_seed):
    """Outputs and input gradients of ``fn(*inputs)`` for a fixed upstream
    gradient."""
    leaves = [t.detach().clone().requires_grad_(t.requires_grad) for t in inputs]
    out = fn(*leaves)
    outs = out if isinstance(out, tuple) else (out,)
    grads = [torch.randn(o.shape, generator=torch.Generator().manual_seed(grad_seed + i))
             .to(o.dtype).to(DEV) for i, o in enumerate(outs)]
    torch.autograd.backward(outs, grads)
    return [o.detach() for o in outs], [None if t.grad is None else t.grad for t in leaves]


def _assert_identical(a, b):
    for x, y in zip(a, b):
        if x is None or y is None:
            assert x is None and y is None
            continue
        assert x.dtype == y.dtype and x.shape == y.shape
        as_int = {torch.bfloat16: torch.int16, torch.float32: torch.int32}
        if x.dtype in as_int:
            x, y = (t.contiguous().view(as_int[t.dtype]) for t in (x, y))
        assert torch.equal(x, y)


def test_rms_linear_lossless(layers_counting):
    require_gpu()
    layers, calls = layers_counting
    buf = _buffer()
    x = _bf16(4, 128, 256, seed=1).requires_grad_()
    w = _bf16(512, 256, seed=2, scale=0.05).requires_grad_()
    gain = (1 + 0.1 * _f32(256, seed=3)).requires_grad_()
    bias = (0.1 * _f32(512, seed=4)).requires_grad_()

    def f(compressed):
        return lambda *t: layers.RMSLinear.apply(*t, buf, compressed, None, 65536)

    dense = _run(f(False), (x, w, gain, bias), 10)
    assert calls == []
    comp = _run(f(True), (x, w, gain, bias), 10)
    assert calls == [(4, 128, 256)]
    _assert_identical(dense[0] + dense[1], comp[0] + comp[1])
    assert all(g is not None for g in comp[1])
    # Below min_elements the input stays dense.
    _run(lambda *t: layers.RMSLinear.apply(*t, buf, True, None, 10 ** 9), (x, w, gain, bias), 10)
    assert len(calls) == 1


def test_rms_norm_qkv_lossless(layers_counting):
    require_gpu()
    layers, calls = layers_counting
    buf = _buffer()
    torch.manual_seed(0)
    q, k, v = (layers.Linear(256, 256).to(DEV) for _ in range(3))
    x = _bf16(2, 256, 256, seed=5).requires_grad_()
    gain = (1 + 0.1 * _f32(256, seed=6)).requires_grad_()

    def run(compressed):
        for m in (q, k, v):
            m.weight.grad = m.bias.grad = None
        outs, grads = _run(lambda x_, g_: layers.rms_norm_qkv(
            x_, g_, q, k, v, buffer=buf, compressed=compressed), (x, gain), 20)
        params = [p.grad.clone() for m in (q, k, v) for p in (m.weight, m.bias)]
        return outs + grads + params

    dense = run(False)
    comp = run(True)
    assert calls == [(2, 256, 256)]
    _assert_identical(dense, comp)


@pytest.mark.parametrize("with_gain", [False, True])
def test_rms_norm_function_lossless(layers_counting, with_gain):
    require_gpu()
    layers, calls = layers_counting
    buf = _buffer()
    x = _bf16(2, 256, 4, 64, seed=7).requires_grad_()
    inputs = (x, (1 + 0.1 * _f32(64, seed=8)).requires_grad_()) if with_gain else (x,)

    def f(compressed):
        if with_gain:
            return lambda x_, g_: layers.RMSNormFunction.apply(x_, g_, buf, compressed, None, 65536)
        return lambda x_: layers.RMSNormFunction.apply(x_, None, buf, compressed, None, 65536)

    dense = _run(f(False), inputs, 30)
    comp = _run(f(True), inputs, 30)
    assert calls == [(2, 256, 4, 64)]
    _assert_identical(dense[0] + dense[1], comp[0] + comp[1])


def test_relu2_linear_lossless(layers_counting):
    require_gpu()
    layers, calls = layers_counting
    buf = _buffer()
    z = _bf16(2, 128, 1024, seed=9).requires_grad_()
    w = _bf16(256, 1024, seed=10, scale=0.03).requires_grad_()
    bias = (0.1 * _f32(256, seed=11)).requires_grad_()

    def f(compressed):
        return lambda *t: layers.Relu2Linear.apply(*t, buf, compressed, None, 65536)

    dense = _run(f(False), (z, w, bias), 40)
    comp = _run(f(True), (z, w, bias), 40)
    assert calls == [(2, 128, 1024)]
    _assert_identical(dense[0] + dense[1], comp[0] + comp[1])


def test_flash_attention_lossless(layers_counting):
    require_gpu()
    layers, calls = layers_counting
    buf = _buffer()
    B, T, H, D = 2, 256, 4, 64
    # BHTD views of BTHD storage, as the model hands them over.
    q, k, v = (_bf16(B, T, H, D, seed=s).transpose(1, 2).requires_grad_() for s in (12, 13, 14))
    w = _bf16(H * D, H * D, seed=15, scale=0.05).requires_grad_()
    bias = (0.1 * _f32(H * D, seed=16)).requires_grad_()

    def run(compressed):
        leaves = [t.detach().transpose(1, 2).clone().transpose(1, 2).requires_grad_()
                  for t in (q, k, v)] + [w.detach().clone().requires_grad_(),
                                         bias.detach().clone().requires_grad_()]
        out = layers.FlashAttention.apply(*leaves, buf, compressed, None, 65536)
        grad = torch.randn(out.shape, generator=torch.Generator().manual_seed(50))
        out.backward(grad.to(out.dtype).to(DEV))
        return [out.detach()] + [t.grad for t in leaves]

    dense = run(False)
    comp = run(True)
    assert calls == [(B, T, H, D)] * 4
    _assert_identical(dense, comp)


def test_compressed_weight_and_embedding():
    require_gpu()
    from losslessly_compressed_tensors_amd.LCTensor import LCTTensor
    from losslessly_compressed_tensors_amd.components import layers
    buf = _buffer()
    torch.manual_seed(1)
    lin_dense = layers.Linear(256, 512).to(DEV)
    lin_comp = layers.Linear(256, 512).to(DEV)
    with torch.no_grad():
        lin_comp.weight.copy_(lin_dense.weight)
        lin_comp.bias.copy_(lin_dense.bias)
    lin_comp.compress_weight(buf)
    assert isinstance(lin_comp.weight, LCTTensor)
    assert torch.equal(layers.dense_weight(lin_comp.weight), lin_dense.weight.detach())
    names = dict(layers.named_trainable_tensors(lin_comp))
    assert set(names) == {"bias", "weight"}

    x = _bf16(4, 128, 256, seed=17)
    gain = torch.ones(256, device=DEV, requires_grad=True)
    results = []
    for lin in (lin_dense, lin_comp):
        xi = x.clone().requires_grad_()
        out = layers.RMSLinear.apply(xi, lin.weight, gain, lin.bias, buf, True, None, 65536)
        out.backward(torch.ones_like(out))
        results.append([out.detach(), xi.grad, lin.weight.grad, lin.bias.grad])
        gain.grad = None
    _assert_identical(*results)

    table = _bf16(1000, 128, seed=18)
    idx = torch.randint(0, 1000, (4, 64), generator=torch.Generator().manual_seed(3)).to(DEV)
    emb = torch.nn.Embedding(1000, 128, dtype=torch.bfloat16).to(DEV)
    with torch.no_grad():
        emb.weight.copy_(table)
    dense_out = layers.Embedding.apply(idx, emb.weight)
    dense_out.backward(torch.ones_like(dense_out))
    layers.compress_weight(emb, buf)
    comp_out = layers.Embedding.apply(idx, emb.weight)
    comp_out.backward(torch.ones_like(comp_out))
    _assert_identical([dense_out.detach()], [comp_out.detach()])
    assert emb.weight.grad is not None
    lin_comp.weight.free()
    emb.weight.free()


def _oracle_mul_add(a, b, alpha, beta=1.0, alpha_is_one=False, beta_is_one=True):
    return oracle.apply_array(oracle.OP_SCALAR_MUL_ADD, bits_of(a), bits_of(b), alpha, beta,
                              alpha_is_one, beta_is_one)


@pytest.mark.parametrize("compressed_weight", [False, True])
def test_sgdm_matches_oracle(compressed_weight):
    require_gpu()
    from losslessly_compressed_tensors_amd.LCTensor import LCTTensor
    from losslessly_compressed_tensors_amd.components.dist_configs import weight_dist
    from losslessly_compressed_tensors_amd.components.sparse_utils import SparseSGDM
    buf = _buffer()
    w0 = _bf16(256, 512, seed=20, scale=0.05)
    p = LCTTensor(w0, buffer=buf, dist=weight_dist) if compressed_weight else w0.clone()
    opt = SparseSGDM([p], lr=0.01, buffer=buf)
    lr = np.float32(-0.01)
    w_bits, m_bits = bits_of(w0), None
    for step in range(3):
        g = _bf16(256, 512, seed=30 + step, scale=0.01)
        p.grad = g
        opt.step()
        g_bits = bits_of(g)
        if m_bits is None:
            m_bits = g_bits
        else:
            m_bits = oracle.apply_array(oracle.OP_SCALAR_MUL_ADD, m_bits, g_bits, 0.9)
        w_bits = oracle.apply_array(oracle.OP_SCALAR_MUL_ADD, m_bits, w_bits, float(lr))
        got_m = bits_of(opt.momentums[0].decompress())
        got_w = bits_of(p.decompress() if compressed_weight else p)
        np.testing.assert_array_equal(got_m, m_bits)
        np.testing.assert_array_equal(got_w, w_bits)
    opt.momentums[0].free()
    if compressed_weight:
        p.free()


def test_muon_compressed_momentum_lossless():
    require_gpu()
    from losslessly_compressed_tensors_amd.components.sparse_utils import SparseMuon
    buf = _buffer()
    w0 = _bf16(256, 768, seed=40, scale=0.05)
    pa, pb = w0.clone(), w0.clone()
    dense = SparseMuon([pa], lr=0.035, weight_decay=0.025, compressed=False, ns_iters=5)
    comp = SparseMuon([pb], lr=0.035, weight_decay=0.025, compressed=True, buffer=buf,
                      zero_first_step=True, ns_iters=5)
    for step in range(3):
        g = _bf16(256, 768, seed=50 + step, scale=0.01)
        pa.grad, pb.grad = g.clone(), g.clone()
        dense.step()
        comp.step()
        assert torch.equal(pa.view(torch.int16), pb.view(torch.int16))
        assert torch.equal(dense.momentums[0].view(torch.int16),
                           comp.momentums[0].decompress().view(torch.int16))
    comp.momentums[0].free()


def test_muon_compressed_weight_matches_oracle():
    require_gpu()
    from losslessly_compressed_tensors_amd.LCTensor import LCTTensor
    from losslessly_compressed_tensors_amd.components.dist_configs import weight_dist
    from losslessly_compressed_tensors_amd.components.sparse_utils import SparseMuon, muon_update
    buf = _buffer()
    w0 = _bf16(512, 256, seed=60, scale=0.05)
    p = LCTTensor(w0, buffer=buf, dist=weight_dist)
    lr, wd = 0.035, 0.025
    opt = SparseMuon([p], lr=lr, weight_decay=wd, compressed=True, buffer=buf, ns_iters=5)
    momentum = torch.zeros_like(w0)
    w_bits = bits_of(w0)
    decay, neg_lr = float(np.float32(1 - lr * wd)), float(np.float32(-lr))
    for step in range(3):
        g = _bf16(512, 256, seed=70 + step, scale=0.01)
        p.grad = g.clone()
        opt.step()
        update = muon_update(g.clone(), momentum, mu=0.95, ns_iters=5)
        w_bits = oracle.apply_array(oracle.OP_SCALAR_MUL_ADD, w_bits, bits_of(update), decay,
                                    neg_lr, False, False)
        np.testing.assert_array_equal(bits_of(p.decompress()), w_bits)
    opt.momentums[0].free()
    p.free()


@pytest.mark.parametrize("compressed_weight", [False, True])
def test_adamw_lossless(compressed_weight):
    require_gpu()
    from losslessly_compressed_tensors_amd.LCTensor import LCTTensor
    from losslessly_compressed_tensors_amd.components.dist_configs import weight_dist
    from losslessly_compressed_tensors_amd.components.sparse_utils import SparseAdamW
    buf = _buffer()
    w0 = _bf16(384, 256, seed=80, scale=0.05)
    pa = w0.clone()
    pb = LCTTensor(w0, buffer=buf, dist=weight_dist) if compressed_weight else w0.clone()
    dense = SparseAdamW([dict(params=[pa], lr=0.01)], compressed=False)
    comp = SparseAdamW([dict(params=[pb], lr=0.01)], compressed=True, buffer=buf)
    for step in range(3):
        g = _bf16(384, 256, seed=90 + step, scale=0.01)
        pa.grad, pb.grad = g.clone(), g.clone()
        dense.step()
        comp.step()
        got = pb.decompress() if compressed_weight else pb
        assert torch.equal(pa.view(torch.int16), got.view(torch.int16))
        state = comp.state[pb]
        assert isinstance(state["exp_avg"], LCTTensor)
        assert torch.equal(dense.state[pa]["exp_avg_sq"].view(torch.int16),
                           state["exp_avg_sq"].decompress().view(torch.int16))


def _tiny(compress_weights, compress_activations, compress_optimizer):
    from examples.nanogpt import train_gpt_lct as gpt
    return gpt.build(torch.device(DEV), compress_weights=compress_weights,
                     compress_activations=compress_activations,
                     compress_optimizer=compress_optimizer, vocab_size=1024, num_layers=2,
                     model_dim=256, head_dim=64, buffer_mib=32, seed=0)


def _steps(model, optimizers, n=3):
    from examples.nanogpt import train_gpt_lct as gpt
    losses = []
    # One batch repeated: the model memorises it, so the loss must fall.
    inputs, targets = gpt.random_tokens(2, 256, DEV, seed=100, token_ids=1000)
    for _ in range(n):
        loss = model(inputs, targets)
        loss.backward()
        for name, p in model.named_trainable_tensors():
            assert p.grad is not None, name
        for opt in optimizers:
            opt.step()
        model.zero_grad()
        losses.append(loss.detach())
    return losses


def _weights(model):
    from losslessly_compressed_tensors_amd.components.layers import dense_weight
    return {name: dense_weight(p).detach().clone() for name, p in model.named_trainable_tensors()}


def test_gpt_compressed_activations_and_momentum_bit_identical():
    """Activations and Muon momentum compressed, weights dense: every loss and
    every final weight equals the uncompressed run's."""
    require_gpu()
    dense_model, dense_opt = _tiny(False, False, False)
    dense_losses = _steps(dense_model, dense_opt)
    dense_weights = _weights(dense_model)
    comp_model, comp_opt = _tiny(False, True, True)
    comp_losses = _steps(comp_model, comp_opt)
    comp_weights = _weights(comp_model)
    for a, b in zip(dense_losses, comp_losses):
        assert torch.equal(a, b)
    assert dense_weights.keys() == comp_weights.keys()
    for name in dense_weights:
        assert torch.equal(dense_weights[name], comp_weights[name]), name
    assert float(dense_losses[-1]) < float(dense_losses[0])


def test_gpt_all_compressed_trains():
    """Weights compressed too: the first loss equals the dense run's (the
    weights decode losslessly); Muon's fused weight update rounds once where
    the dense path rounds twice, so later steps are only required to train."""
    require_gpu()
    from losslessly_compressed_tensors_amd.LCTensor import LCTTensor
    from losslessly_compressed_tensors_amd.tensor_buffer import verify_buffer
    dense_model, dense_opt = _tiny(False, False, False)
    dense_losses = _steps(dense_model, dense_opt)
    model, opt = _tiny(True, True, True)
    assert isinstance(model.blocks[0].attn.q.weight, LCTTensor)
    losses = _steps(model, opt)
    assert torch.equal(losses[0], dense_losses[0])
    assert all(torch.isfinite(l) for l in losses)
    assert float(losses[-1]) < float(losses[0])
    verify_buffer(model.tensor_buffer)


# ---------------------------------------------------------------------------
# Config 5 at its stated shape: 12 layers, width 768, 12 heads, vocabulary
# 50304 (ids below 50257), sequence 1024, batch 8
# (examples/nanogpt/train_gpt_lct.py:86-303 of the reference).
# ---------------------------------------------------------------------------


def _full(compress_weights, compress_activations, compress_optimizer):
    from examples.nanogpt import train_gpt_lct as gpt
    model, optimizers = gpt.build(torch.device(DEV), compress_weights=compress_weights,
                                  compress_activations=compress_activations,
                                  compress_optimizer=compress_optimizer, seed=0)
    assert (len(model.blocks), model.embed.weight.shape) == (12, (50304, 768))
    assert model.blocks[0].attn.num_heads == 12
    return gpt, model, optimizers


def _full_steps(gpt, model, optimizers, steps):
    losses = []
    for step in range(steps):
        inputs, targets = gpt.random_tokens(gpt.BATCH, gpt.SEQ_LEN, DEV, seed=500 + step)
        assert inputs.shape == (8, 1024) and int(inputs.max()) < 50257
        losses.append(gpt.train_step(model, optimizers, inputs, targets))
        print(f"config 5 step {step}: loss {float(losses[-1]):.1f}", flush=True)
    return losses


def test_config5_full_shape_compressed_activations_and_momentum_bit_identical(
        layers_counting):
    """Two GPT-2-small steps with activations and Muon momentum compressed give
    every loss and every final weight of the uncompressed run, bit for bit."""
    require_gpu()
    print("case config 5 dense", flush=True)
    gpt, model, optimizers = _full(False, False, False)
    dense_losses = _full_steps(gpt, model, optimizers, 2)
    dense_weights = _weights(model)
    del model, optimizers
    torch.cuda.empty_cache()
    print("case config 5 activations + momentum compressed", flush=True)
    _, calls = layers_counting
    gpt, model, optimizers = _full(False, True, True)
    losses = _full_steps(gpt, model, optimizers, 2)
    weights = _weights(model)
    from losslessly_compressed_tensors_amd.LCTensor import LCTTensor
    from losslessly_compressed_tensors_amd.tensor_buffer import verify_buffer
    assert len(calls) > 100, "the layers' compressed branch did not run"
    assert all(isinstance(m, LCTTensor) for m in optimizers[1].momentums)
    for a, b in zip(dense_losses, losses):
        assert torch.equal(a, b)
    assert dense_weights.keys() == weights.keys()
    for name in dense_weights:
        _assert_identical([dense_weights[name]], [weights[name]])
    verify_buffer(model.tensor_buffer)


def test_config5_full_shape_all_compressed_weight_update_matches_oracle(monkeypatch):
    """Weights, activations and momentum compressed: the first loss equals the
    dense run's (the weights decode losslessly), and the fused Muon update of
    a block matrix, p <- fma(p, 1 - lr wd, fl(-lr u)) rounded once, equals
    the oracle's arithmetic element by element."""
    require_gpu()
    from losslessly_compressed_tensors_amd.components import sparse_utils
    from losslessly_compressed_tensors_amd.LCTensor import LCTTensor
    from losslessly_compressed_tensors_amd.tensor_buffer import verify_buffer
    print("case config 5 dense first loss", flush=True)
    gpt, model, optimizers = _full(False, False, False)
    dense_first = _full_steps(gpt, model, optimizers, 1)[0]
    del model, optimizers
    torch.cuda.empty_cache()
    print("case config 5 all compressed", flush=True)
    gpt, model, optimizers = _full(True, True, True)
    # Every projection (the head's included) starts at zero, so the first
    # step's gradients reach no block matrix; on the second step the output
    # projections take a full update, while q and fc (behind the still-zero
    # projections) take only the decay, which rounds away in BF16.  The tall
    # fc matrix is transposed into the wide group.
    losses = _full_steps(gpt, model, optimizers, 1)
    assert torch.equal(losses[0], dense_first)
    watched = {"blocks.0.mlp.proj.weight": model.blocks[0].mlp.proj.weight,
               "blocks.11.attn.proj.weight": model.blocks[11].attn.proj.weight,
               "blocks.5.mlp.fc.weight": model.blocks[5].mlp.fc.weight,
               "blocks.3.attn.q.weight": model.blocks[3].attn.q.weight}
    assert all(isinstance(p, LCTTensor) for p in watched.values())
    before = {name: bits_of(p.decompress()) for name, p in watched.items()}
    seen = {}
    real_apply_many = sparse_utils.SparseMuon._apply_many

    def recording_apply_many(self, params, updates):
        for param, update in zip(params, updates):
            for name, p in watched.items():
                if param is p:
                    seen[name] = bits_of(update)
        return real_apply_many(self, params, updates)

    monkeypatch.setattr(sparse_utils.SparseMuon, "_apply_many", recording_apply_many)
    _full_steps(gpt, model, optimizers, 1)
    muon = optimizers[1]
    decay = float(np.float32(1 - muon.lr * muon.weight_decay))
    neg_lr = float(np.float32(-muon.lr))
    for name, p in watched.items():
        expect = oracle.apply_array(oracle.OP_SCALAR_MUL_ADD, before[name], seen[name], decay,
                                    neg_lr, False, False)
        np.testing.assert_array_equal(bits_of(p.decompress()), expect, err_msg=name)
        if name.endswith("proj.weight"):
            assert not np.array_equal(expect, before[name]), name
    verify_buffer(model.tensor_buffer)
