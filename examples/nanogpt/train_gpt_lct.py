"""GPT-2-small-shaped training step with weights, activations and Muon momentum
held compressed (``examples/nanogpt/train_gpt_lct.py`` of the reference).

The model, initialisation, loss and optimizer split follow the reference
trainer (``train_gpt_lct.py:86-353``): pre-norm blocks with one shared RMSNorm
per Q/K/V, RMS-normalised Q and K, half-truncated rotary embeddings, causal
flash attention with scale 0.12, a squared-ReLU MLP, a soft-capped
cross-entropy head evaluated in checkpointed chunks of 4096 tokens, AdamW for
the embedding, the head and the vectors, and Muon (12 Newton-Schulz
iterations, compressed momentum) for the block matrices.

Differences, all deliberate: token ids are uniform random on the device (no
FineWeb shards, no network); the dense regions run eagerly, without a
tracing compiler; one step is one microbatch of ``batch`` sequences.

``python examples/nanogpt/train_gpt_lct.py --mode both`` prints, per mode,
tokens per second and peak device memory of the training step.
"""
from __future__ import annotations

import argparse
import json
import sys
import time
from pathlib import Path

if __package__ in (None, ""):
    sys.path.insert(0, str(Path(__file__).resolve().parents[2]))

import torch
import torch.nn.functional as F
from torch import Tensor, nn
from torch.utils.checkpoint import checkpoint

from losslessly_compressed_tensors_amd.comp_format import Distribution, DistType, NoiseLevel
from losslessly_compressed_tensors_amd.LCTensor import LCTTensor
from losslessly_compressed_tensors_amd.components.layers import (
    Embedding, FlashAttention, Linear, RMSLinear, RMSNormFunction, Relu2Linear,
    compress_weight, dense_weight, flush_saved, named_trainable_tensors, prefetch_saved,
    prefetch_weights, queued_saved, rms_norm_qkv,
)
from losslessly_compressed_tensors_amd.components.sparse_utils import SparseAdamW, SparseMuon
from losslessly_compressed_tensors_amd.tensor_buffer import TensorBuffer, _free_regions_snapshot

# Codebooks of the nanoGPT trainer (examples/nanogpt/dist_configs.py:4-7 of the
# reference): they differ from the training integration's defaults in the
# weights' zero mass and the post-ReLU layout.
weight_dist = Distribution(DistType.LAPLACE, noise_level=NoiseLevel.CLEAN, zero_prob=0.01)
momentum_dist = Distribution(DistType.EMPIRICAL, noise_level=NoiseLevel.CLEAN, zero_prob=0.02)
act_dist = Distribution(DistType.LAPLACE, noise_level=NoiseLevel.CLEAN)
act_relu_dist = Distribution(DistType.LAPLACE, noise_level=NoiseLevel.SPARSE, zero_prob=0.5)

# GPT-2-small shape: 12 layers, width 768, 12 heads of 64; the embedding and
# head padded to 50304 rows (a multiple of 128) as in the reference trainer,
# with token ids drawn from GPT-2's 50257.
VOCAB_SIZE = 50304
TOKEN_IDS = 50257
NUM_LAYERS = 12
MODEL_DIM = 768
HEAD_DIM = 64
SEQ_LEN = 1024
BATCH = 8
CHUNK_TOKENS = 4096
BUFFER_SIZE_MIB = 64
MIN_COMPRESS_ELEMENTS = 65536
SOFTCAP = 15.0


class SoftcapCrossEntropy(torch.autograd.Function):
    """Summed cross-entropy of ``15 x / sqrt(x^2 + 225)``-capped logits; saves
    the BF16 logits and the row log-sum-exp (train_gpt_lct.py:88-140)."""

    @staticmethod
    def head_loss(x, targets, weight, gains, bias, buffer, compressed, min_elements,
                  checkpoint_head=True):
        W = dense_weight(weight)

        def project_and_loss(chunk, chunk_targets):
            # A checkpointed chunk is consumed at once: its input stays dense.
            logits = RMSLinear.apply(
                chunk, weight, gains, bias, buffer,
                compressed and torch.is_grad_enabled() and not checkpoint_head,
                act_dist, min_elements, W)
            return SoftcapCrossEntropy.apply(logits, chunk_targets)

        if not checkpoint_head:
            return project_and_loss(x, targets)
        x = x.reshape(-1, x.shape[-1])
        targets = targets.reshape(-1)
        loss = x.new_zeros((), dtype=torch.float32)
        for start in range(0, targets.numel(), CHUNK_TOKENS):
            chunk, chunk_targets = x[start:start + CHUNK_TOKENS], targets[start:start + CHUNK_TOKENS]
            if torch.is_grad_enabled():
                loss = loss + checkpoint(project_and_loss, chunk, chunk_targets,
                                         use_reentrant=True, preserve_rng_state=False)
            else:
                loss = loss + project_and_loss(chunk, chunk_targets)
        return loss

    # Rows of a chunk evaluated together: every quantity is per row (the
    # log-sum-exp) or per element, so row groups give each row's values
    # exactly; groups keep the FP32 temporaries of the eager evaluation to
    # 512 x vocab elements where the reference fuses them with torch.compile.
    ROWS = 512

    @staticmethod
    def forward(ctx, logits: Tensor, targets: Tensor):
        rows = logits.reshape(targets.numel(), -1)
        flat_targets = targets.reshape(-1, 1)
        logsumexp = torch.empty((rows.shape[0], 1), dtype=torch.float32, device=logits.device)
        loss = torch.zeros((), dtype=torch.float32, device=logits.device)
        for start in range(0, rows.shape[0], SoftcapCrossEntropy.ROWS):
            end = start + SoftcapCrossEntropy.ROWS
            x = rows[start:end].float()
            capped = SOFTCAP * x * (x.square() + SOFTCAP ** 2).rsqrt()
            lse = capped.logsumexp(dim=-1, keepdim=True)
            logsumexp[start:end] = lse
            loss += (lse - capped.gather(1, flat_targets[start:end])).sum()
        ctx.save_for_backward(logits, targets, logsumexp)
        return loss

    @staticmethod
    def backward(ctx, grad_output):
        logits, targets, logsumexp = ctx.saved_tensors
        rows = logits.reshape(targets.numel(), -1)
        flat_targets = targets.reshape(-1, 1)
        grad = torch.empty_like(rows)
        columns = torch.arange(rows.shape[-1], device=logits.device)
        for start in range(0, rows.shape[0], SoftcapCrossEntropy.ROWS):
            end = start + SoftcapCrossEntropy.ROWS
            x = rows[start:end].float()
            inv = (x.square() + SOFTCAP ** 2).rsqrt()
            probabilities = (SOFTCAP * x * inv - logsumexp[start:end]).exp()
            is_target = columns == flat_targets[start:end]
            # d/dx [15 x (x^2 + 225)^-1/2] = 15^3 (x^2 + 225)^-3/2.
            grad[start:end] = ((probabilities - is_target.to(x.dtype)) * inv.pow(3)
                               * SOFTCAP ** 3 * grad_output)
        return grad.reshape(logits.shape), None


class RMSNorm(nn.Module):
    def __init__(self, dim):
        super().__init__()
        self.gains = nn.Parameter(torch.ones(dim))


class Rotary(nn.Module):
    """Rotary embedding on the first half of each head's channels; the second
    half's frequencies are zero (train_gpt_lct.py:150-165)."""

    def __init__(self, dim: int):
        super().__init__()
        freq = (1 / 1024) ** torch.linspace(0, 1, steps=dim // 4, dtype=torch.float32)
        self.register_buffer("angular_freq", torch.cat([freq, freq.new_zeros(dim // 4)]))

    def forward(self, x_BTHD: Tensor):
        pos = torch.arange(x_BTHD.size(1), dtype=torch.float32, device=x_BTHD.device)
        theta = torch.outer(pos, self.angular_freq)[None, :, None, :]
        cos, sin = theta.cos(), theta.sin()
        x1, x2 = x_BTHD.float().chunk(2, dim=-1)
        return torch.cat((x1 * cos + x2 * sin, x2 * cos - x1 * sin), 3).type_as(x_BTHD)


class CausalSelfAttention(nn.Module):
    def __init__(self, dim: int, head_dim=HEAD_DIM, compress_activations=False,
                 min_compress_elements=MIN_COMPRESS_ELEMENTS):
        super().__init__()
        if dim % head_dim:
            raise ValueError("model_dim must be divisible by head_dim")
        self.compress_activations = compress_activations
        self.min_compress_elements = min_compress_elements
        self.tensor_buffer = None
        self.num_heads, self.head_dim = dim // head_dim, head_dim
        hdim = self.num_heads * head_dim
        self.q, self.k, self.v = Linear(dim, hdim), Linear(dim, hdim), Linear(dim, hdim)
        self.proj = Linear(hdim, dim)
        self.rotary = Rotary(head_dim)

    def forward(self, x: Tensor, norm_weight: Tensor):
        B, T = x.size(0), x.size(1)
        compressed = self.compress_activations and torch.is_grad_enabled()
        q, k, v = rms_norm_qkv(x, norm_weight, self.q, self.k, self.v, buffer=self.tensor_buffer,
                               compressed=compressed, distribution=act_dist,
                               min_elements=self.min_compress_elements)
        shape = (B, T, self.num_heads, self.head_dim)
        q, k, v = q.view(shape), k.view(shape), v.view(shape)
        norm_args = (None, self.tensor_buffer, compressed, act_dist, self.min_compress_elements)
        q = self.rotary(RMSNormFunction.apply(q, *norm_args))
        k = self.rotary(RMSNormFunction.apply(k, *norm_args))
        return FlashAttention.apply(q.transpose(1, 2), k.transpose(1, 2), v.transpose(1, 2),
                                    self.proj.weight, self.proj.bias, self.tensor_buffer,
                                    compressed, act_dist, self.min_compress_elements)


class MLP(nn.Module):
    def __init__(self, dim: int, compress_activations=False,
                 min_compress_elements=MIN_COMPRESS_ELEMENTS):
        super().__init__()
        self.compress_activations = compress_activations
        self.min_compress_elements = min_compress_elements
        self.tensor_buffer = None
        self.fc, self.proj = Linear(dim, 4 * dim), Linear(4 * dim, dim)

    def forward(self, x: Tensor, norm_weight: Tensor):
        compressed = self.compress_activations and torch.is_grad_enabled()
        z = RMSLinear.apply(x, self.fc.weight, norm_weight, self.fc.bias, self.tensor_buffer,
                            compressed, act_dist, self.min_compress_elements)
        return Relu2Linear.apply(z, self.proj.weight, self.proj.bias, self.tensor_buffer,
                                 compressed, act_relu_dist, self.min_compress_elements)


class Block(nn.Module):
    def __init__(self, dim: int, head_dim=HEAD_DIM, compress_activations=False,
                 min_compress_elements=MIN_COMPRESS_ELEMENTS):
        super().__init__()
        self.attn = CausalSelfAttention(dim, head_dim, compress_activations, min_compress_elements)
        self.mlp = MLP(dim, compress_activations, min_compress_elements)
        self.norm1, self.norm2 = RMSNorm(dim), RMSNorm(dim)

    def weights(self):
        attn, mlp = self.attn, self.mlp
        return [attn.q.weight, attn.k.weight, attn.v.weight, attn.proj.weight, mlp.fc.weight,
                mlp.proj.weight]

    def forward(self, x: Tensor):
        # The block's compressed weights are decoded together, once before its
        # forward and once when its backward starts (the hook on its output),
        # instead of one decode launch per use.
        # Likewise the activations the attention and the MLP save: compressed
        # together when the block's forward ends (flush_saved), decoded part by
        # part when that part's backward starts (the hooks on the parts'
        # outputs).
        weights = self.weights()
        prefetch_weights(weights)
        a = self.attn(x, self.norm1.gains)
        saved_attn = queued_saved()
        x = x + a
        m = self.mlp(x, self.norm2.gains)
        attn_ids = {id(s) for s in saved_attn}
        saved_mlp = [s for s in flush_saved() if id(s) not in attn_ids]
        out = x + m
        if out.requires_grad:
            if any(isinstance(w, LCTTensor) for w in weights):
                out.register_hook(lambda grad: prefetch_weights(self.weights()))
            if saved_attn:
                a.register_hook(lambda grad: prefetch_saved(saved_attn))
            if saved_mlp:
                m.register_hook(lambda grad: prefetch_saved(saved_mlp))
        return out


class GPT(nn.Module):
    def __init__(self, vocab_size=VOCAB_SIZE, num_layers=NUM_LAYERS, model_dim=MODEL_DIM,
                 head_dim=HEAD_DIM, compress_activations=False,
                 min_compress_elements=MIN_COMPRESS_ELEMENTS):
        super().__init__()
        self.embed = nn.Embedding(vocab_size, model_dim, dtype=torch.bfloat16)
        self.blocks = nn.ModuleList([Block(model_dim, head_dim, compress_activations,
                                           min_compress_elements) for _ in range(num_layers)])
        self.compress_activations = compress_activations
        self.min_compress_elements = min_compress_elements
        self.proj = Linear(model_dim, vocab_size)
        self.norm1, self.norm2 = RMSNorm(model_dim), RMSNorm(model_dim)
        self.tensor_buffer = None

    def set_tensor_buffer(self, buffer):
        self.tensor_buffer = buffer
        for block in self.blocks:
            block.mlp.tensor_buffer = block.attn.tensor_buffer = buffer

    def compress_weights(self):
        for module in self.modules():
            if isinstance(module, (Linear, nn.Embedding)):
                compress_weight(module, self.tensor_buffer, distribution=weight_dist)

    def named_trainable_tensors(self):
        return named_trainable_tensors(self)

    def zero_grad(self, set_to_none=True):
        for _, p in self.named_trainable_tensors():
            p.grad = None

    def forward(self, inputs: Tensor, targets: Tensor):
        compressed = self.compress_activations and torch.is_grad_enabled()
        x = RMSNormFunction.apply(Embedding.apply(inputs, self.embed.weight), self.norm1.gains,
                                  self.tensor_buffer, compressed, act_dist,
                                  self.min_compress_elements)
        for block in self.blocks:
            x = block(x)
        return SoftcapCrossEntropy.head_loss(x, targets, self.proj.weight, self.norm2.gains,
                                             self.proj.bias, self.tensor_buffer,
                                             self.compress_activations, self.min_compress_elements)


def initialize_model(model):
    """Zero projections and biases, N(0,1) embedding, N(0, 0.33/fan_in) other
    matrices, unit gains (train_gpt_lct.py:315-330), before any compression."""
    with torch.no_grad():
        for name, p in model.named_parameters():
            if name.endswith("weight"):
                if "proj" in name:
                    p.zero_()
                elif "embed" in name:
                    p.normal_()
                else:
                    p.normal_(std=0.33 ** 0.5 / p.size(-1) ** 0.5)
            elif name.endswith("bias"):
                p.zero_()
            elif name.endswith("gains"):
                p.fill_(1)
            else:
                raise ValueError(f"Uninitialized parameter: {name}")


def make_optimizers(model, compressed=False):
    """AdamW for the embedding, the head and the vectors; Muon for the block
    matrices (train_gpt_lct.py:333-348)."""
    named = dict(model.named_trainable_tensors())
    adam = SparseAdamW([
        dict(params=[named["embed.weight"]], lr=0.3),
        dict(params=[named["proj.weight"]], lr=1 / 320),
        dict(params=[p for p in named.values() if p.ndim < 2], lr=0.01),
    ], compressed=False, buffer=model.tensor_buffer)
    muon = SparseMuon([p for name, p in named.items() if name.startswith("blocks.") and p.ndim >= 2],
                      lr=0.035, weight_decay=0.025, compressed=compressed,
                      buffer=model.tensor_buffer, distribution=momentum_dist,
                      zero_first_step=True, ns_iters=12)
    parameters = [p for g in adam.param_groups for p in g["params"]] + muon.params
    assert len(parameters) == len(named)
    assert {id(p) for p in parameters} == {id(p) for p in named.values()}
    return adam, muon


def build(device, *, compress_weights, compress_activations, compress_optimizer,
          use_buffer=True, vocab_size=VOCAB_SIZE, num_layers=NUM_LAYERS, model_dim=MODEL_DIM,
          head_dim=HEAD_DIM, buffer_mib=BUFFER_SIZE_MIB, seed=0):
    """Model and optimizers for one mode, initialised from ``seed``."""
    torch.manual_seed(seed)
    model = GPT(vocab_size, num_layers, model_dim, head_dim,
                compress_activations=compress_activations).to(device)
    initialize_model(model)
    if use_buffer and (compress_weights or compress_activations or compress_optimizer):
        model.set_tensor_buffer(TensorBuffer(buffer_mib * 2 ** 20, device=device))
    if compress_weights:
        model.compress_weights()
    return model, make_optimizers(model, compressed=compress_optimizer)


def random_tokens(batch, seq_len, device, seed, token_ids=TOKEN_IDS):
    """Uniform token ids and their next-token targets, drawn on the CPU."""
    g = torch.Generator().manual_seed(seed)
    window = torch.randint(0, token_ids, (batch, seq_len + 1), generator=g)
    return (window[:, :-1].to(device=device, dtype=torch.int32),
            window[:, 1:].to(device=device, dtype=torch.int64))


def train_step(model, optimizers, inputs, targets):
    """Forward, backward and both optimizer steps; returns the summed loss."""
    loss = model(inputs, targets)
    loss.backward()
    for opt in optimizers:
        opt.step()
    model.zero_grad(set_to_none=True)
    return loss.detach()


def resident_bytes(model, optimizers) -> int:
    """Bytes of weights (compressed size for ``LCTTensor``s) and Muon momentum."""
    total = 0
    for _, p in model.named_trainable_tensors():
        total += p.nbytes if hasattr(p, "x") else p.numel() * p.element_size()
    for m in optimizers[1].momentums:
        if m is not None:
            total += m.nbytes if hasattr(m, "x") else m.numel() * m.element_size()
    return total


def measure(device, *, compressed: bool, steps: int, warmup: int, batch=BATCH, seq_len=SEQ_LEN,
            **shape):
    """Tokens per second and peak allocated bytes of ``steps`` timed steps.
    The peak counts what the model, its optimizers and the steps allocate:
    memory the caller held before the call is subtracted."""
    held_before = torch.cuda.memory_allocated(device)
    model, optimizers = build(device, compress_weights=compressed,
                              compress_activations=compressed,
                              compress_optimizer=compressed, **shape)
    losses = []
    for i in range(warmup):
        inputs, targets = random_tokens(batch, seq_len, device, seed=1000 + i)
        losses.append(train_step(model, optimizers, inputs, targets))
    batches = [random_tokens(batch, seq_len, device, seed=2000 + i) for i in range(steps)]
    torch.cuda.synchronize(device)
    resident = resident_bytes(model, optimizers)
    torch.cuda.reset_peak_memory_stats(device)
    start = time.perf_counter()
    for inputs, targets in batches:
        losses.append(train_step(model, optimizers, inputs, targets))
    torch.cuda.synchronize(device)
    elapsed = time.perf_counter() - start
    peak = torch.cuda.max_memory_allocated(device) - held_before
    result = {
        "tokens_per_s": round(steps * batch * seq_len / elapsed, 1),
        "ms_per_step": round(1e3 * elapsed / steps, 3),
        "peak_allocated_mib": round(peak / 2 ** 20, 1),
        "resident_state_mib": round(resident / 2 ** 20, 1),
        "final_loss_per_token": round(float(losses[-1]) / (batch * seq_len), 5),
    }
    if model.tensor_buffer is not None:
        buffer = model.tensor_buffer
        free = sum(size for _, size in _free_regions_snapshot(buffer))
        result["buffer_used_mib"] = round((buffer.capacity_bytes - free) / 2 ** 20, 2)
    del model, optimizers
    torch.cuda.empty_cache()
    return result


def main():
    parser = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    parser.add_argument("--mode", choices=("lct", "dense", "both"), default="both")
    parser.add_argument("--steps", type=int, default=10)
    parser.add_argument("--warmup", type=int, default=3)
    parser.add_argument("--batch", type=int, default=BATCH)
    parser.add_argument("--layers", type=int, default=NUM_LAYERS)
    args = parser.parse_args()
    if not torch.cuda.is_available():
        raise RuntimeError("training needs a GPU")
    device = torch.device("cuda:0")
    torch.cuda.set_device(device)
    modes = ("dense", "lct") if args.mode == "both" else (args.mode,)
    for mode in modes:
        result = measure(device, compressed=mode == "lct", steps=args.steps, warmup=args.warmup,
                         batch=args.batch, num_layers=args.layers)
        print(json.dumps({"mode": mode, **result}), flush=True)


if __name__ == "__main__":
    main()
