"""Autograd layers that keep what backward needs compressed.

Same operators, argument order and gradients as ``LCT/components/layers.py``:
each ``torch.autograd.Function`` runs its dense math on the device's libraries
(hipBLASLt GEMMs, ATen's fused RMSNorm and flash attention), and between
forward and backward holds its saved activation as a ``CompressedTensor``
(when ``compressed`` and the tensor has at least ``min_elements`` elements),
decoding and freeing it once in backward.  Weights may be ``LCTTensor``s
(``compress_weight``): every use decodes them.  The codec is lossless, so a
compressed layer's outputs and gradients are bit-identical to the same layer
without compression.

The reference wraps the dense regions in ``torch.compile``; here they run
eagerly (no tracing compiler or generated kernels), in the same arithmetic
order, so compressed and uncompressed runs of this module agree bit for bit.
"""
from __future__ import annotations

import torch
import torch.nn.functional as F
from torch import Tensor, nn

from ..LCTensor import LCTTensor
from ..codec.decode import decode_batch
from ..operations import compress, compress_batch, decompress
from .dist_configs import act_dist, act_relu_dist, weight_dist
from .ops import rms_norm, rms_norm_backward

__all__ = [
    "dense_weight", "prefetch_weights", "RMSLinear", "rms_norm_qkv", "RMSNormFunction",
    "Relu2Linear", "FlashAttention", "compress_weight", "Linear", "Embedding",
    "named_trainable_tensors", "flush_saved", "queued_saved", "prefetch_saved",
    "batch_saved_compression",
]

# Causal attention scale of the trainer (LCT/components/layers.py:232-236).
ATTENTION_SCALE = 0.12


# Dense copies of compressed weights decoded ahead of their use, keyed by the
# LCTTensor's id: (the CompressedTensor decoded, its dense copy).  Each copy is
# handed to the next dense_weight() of its weight and dropped.
_prefetched: dict[int, tuple] = {}


def prefetch_weights(weights) -> None:
    """Decode the compressed ones among ``weights`` in as few launches as
    possible (``decode_batch``: one per 16 tensors), for their next
    ``dense_weight``.  A block's weights are a few codec blocks each, so one
    decode each would be bound by one block's latency per tensor."""
    pending = [w for w in weights if isinstance(w, LCTTensor)]
    if not pending:
        return
    for w, dense in zip(pending, decode_batch([w.x for w in pending])):
        _prefetched[id(w)] = (w.x, dense)


def dense_weight(weight):
    """The weight as a dense BF16 tensor (decoded if it is an ``LCTTensor``:
    the copy ``prefetch_weights`` made of its current value, or a decode now)."""
    if not isinstance(weight, LCTTensor):
        return weight
    entry = _prefetched.pop(id(weight), None)
    if entry is not None and entry[0] is weight.x:
        return entry[1]
    return weight.decompress()


# Saved activations wait here, dense, until they can be compressed together:
# flush_saved() compresses the queue with one launch per 16 tensors
# (compress_batch), and runs when the queue is full, when a queued tensor is
# taken, and wherever a caller ends a group (a block's attention or MLP).  A
# layer's activations are a few codec blocks per tensor, so one compress
# launch each would be bound by one block's latency.
_MAX_QUEUE = 16
_queue: list["_SavedActivation"] = []
_batching = {"enabled": True}


def batch_saved_compression(enabled: bool) -> bool:
    """Queue saved activations for batched compression (``True``, the default)
    or compress each in its layer's forward; returns the previous setting.
    The compressed records are the same either way."""
    previous, _batching["enabled"] = _batching["enabled"], bool(enabled)
    if not enabled:
        flush_saved()
    return previous


def flush_saved() -> list:
    """Compress the queued saved activations and return them (one
    ``compress_batch`` per buffer).  A queued tensor modified in place since
    it was saved raises, as autograd's saved-tensor check would."""
    global _queue
    queued, _queue = _queue, []
    by_buffer: dict[int, list] = {}
    for saved in queued:
        if saved.value._version != saved.version:
            raise RuntimeError(
                "a tensor saved for backward was modified in place before it was compressed")
        by_buffer.setdefault(id(saved.buffer), []).append(saved)
    for members in by_buffer.values():
        values = compress_batch([s.value for s in members], [s.distribution for s in members],
                                buffer=members[0].buffer)
        for saved, value in zip(members, values):
            saved.value, saved.queued, saved.distribution, saved.buffer = value, False, None, None
    return queued


def queued_saved() -> list:
    """The saved activations waiting for the next ``flush_saved`` (a copy of
    the queue): a caller that compresses two groups in one launch keeps the
    first group's members apart with it."""
    return list(_queue)


def prefetch_saved(saved) -> None:
    """Decode the still-compressed members of ``saved`` (the list a
    ``flush_saved`` returned) with one launch per 16 (``decode_batch``) and
    free their storage; each one's ``take()`` then returns its dense copy."""
    pending = [s for s in saved if s.compressed and s.value is not None and not s.queued]
    if not pending:
        return
    for s, dense in zip(pending, decode_batch([s.value for s in pending])):
        s.value.free()
        s.value, s.compressed = dense, False


class _SavedActivation:
    """One saved tensor, compressed into ``buffer`` or kept as is."""

    __slots__ = ("value", "compressed", "queued", "version", "distribution", "buffer")

    def __init__(self, tensor: Tensor, compressed: bool, distribution, buffer):
        self.compressed = compressed
        self.queued = False
        self.value = tensor
        if not compressed:
            return
        if _batching["enabled"] and buffer is not None and tensor.is_cuda:
            self.queued, self.version = True, tensor._version
            self.distribution, self.buffer = distribution, buffer
            _queue.append(self)
            if len(_queue) >= _MAX_QUEUE:
                flush_saved()
        else:
            self.value = compress(tensor, distribution=distribution, buffer=buffer)

    def take(self) -> Tensor:
        """The saved tensor; a compressed one is decoded and its storage freed."""
        if self.queued:
            flush_saved()
        value, self.value = self.value, None
        if not self.compressed:
            return value
        dense = decompress(value)
        value.free()
        return dense


def _normalized(x: Tensor, rstd: Tensor, gain: Tensor) -> Tensor:
    """RMSNorm output rebuilt from the saved reciprocal RMS: the gain applied in
    FP32, one rounding to BF16 (LCT/components/layers.py:16-19)."""
    return (x.float() * rstd * gain.float()).to(x.dtype).reshape(-1, x.shape[-1])


class RMSLinear(torch.autograd.Function):
    """RMSNorm then one projection; saves only the norm input
    (LCT/components/layers.py:22-71)."""

    @staticmethod
    def forward(ctx, x, weight, norm_weight, bias, buffer=None, compressed=False,
                distribution=None, min_elements=65536, decoded_weight=None):
        W = dense_weight(weight) if decoded_weight is None else decoded_weight
        normalized, rstd = rms_norm(x, norm_weight.to(x.dtype))
        output = F.linear(normalized, W, bias.to(x.dtype))
        del normalized
        ctx.saved = _SavedActivation(x, compressed and x.numel() >= min_elements,
                                     distribution or act_dist, buffer)
        ctx.save_for_backward(norm_weight, rstd, weight if decoded_weight is None else decoded_weight)
        ctx.bias_dtype = bias.dtype
        return output

    @staticmethod
    def backward(ctx, grad):
        norm_weight, rstd, weight = ctx.saved_tensors
        x = ctx.saved.take()
        ctx.saved = None
        W = dense_weight(weight)
        gain = norm_weight.to(x.dtype)
        g = grad.reshape(-1, grad.shape[-1])
        grad_x, grad_gain = rms_norm_backward((g @ W).reshape(x.shape), x, rstd, gain)
        grad_weight = g.T @ _normalized(x, rstd, gain)
        grad_bias = g.sum(0).to(ctx.bias_dtype)
        return (grad_x, grad_weight, grad_gain.to(norm_weight.dtype), grad_bias,
                None, None, None, None, None)


class _RMSNormQKV(torch.autograd.Function):
    """One RMSNorm shared by the Q, K and V projections, one saved input
    (LCT/components/layers.py:74-129)."""

    @staticmethod
    def forward(ctx, x, norm_weight, buffer, compressed, distribution,
                q_weight, q_bias, k_weight, k_bias, v_weight, v_bias):
        weights = (q_weight, k_weight, v_weight)
        biases = (q_bias, k_bias, v_bias)
        normalized, rstd = rms_norm(x, norm_weight.to(x.dtype))
        outputs = tuple(F.linear(normalized, dense_weight(w), b.to(x.dtype))
                        for w, b in zip(weights, biases))
        del normalized
        ctx.saved = _SavedActivation(x, compressed, distribution, buffer)
        ctx.save_for_backward(norm_weight, rstd, *weights)
        ctx.bias_dtypes = tuple(b.dtype for b in biases)
        return outputs

    @staticmethod
    def backward(ctx, grad_q, grad_k, grad_v):
        norm_weight, rstd, *weights = ctx.saved_tensors
        x = ctx.saved.take()
        ctx.saved = None
        gain = norm_weight.to(x.dtype)
        grads = [g.reshape(-1, g.shape[-1]) for g in (grad_q, grad_k, grad_v)]
        dense = [dense_weight(w) for w in weights]
        # V first, then K, then Q, accumulated in place.
        grad_normalized = grads[2] @ dense[2]
        grad_normalized.add_(grads[1] @ dense[1])
        grad_normalized.add_(grads[0] @ dense[0])
        grad_x, grad_gain = rms_norm_backward(grad_normalized.reshape(x.shape), x, rstd, gain)
        del grad_normalized, dense
        normalized = _normalized(x, rstd, gain)
        parameter_grads = []
        for g, bias_dtype in zip(grads, ctx.bias_dtypes):
            parameter_grads += [g.T @ normalized, g.sum(0).to(bias_dtype)]
        return (grad_x, grad_gain.to(norm_weight.dtype), None, None, None, *parameter_grads)


def rms_norm_qkv(x, norm_weight, q, k, v, *, buffer=None, compressed=False,
                 distribution=None, min_elements=65536):
    """Normalise ``x`` once and project it with the ``Linear`` modules ``q``,
    ``k``, ``v`` (LCT/components/layers.py:132-137)."""
    return _RMSNormQKV.apply(x, norm_weight, buffer, compressed and x.numel() >= min_elements,
                             distribution or act_dist, q.weight, q.bias, k.weight, k.bias,
                             v.weight, v.bias)


class RMSNormFunction(torch.autograd.Function):
    """RMSNorm with an optional gain and an optionally compressed saved input
    (LCT/components/layers.py:140-176)."""

    @staticmethod
    def forward(ctx, x, gains, buffer, compressed, distribution, min_elements):
        output, rstd = rms_norm(x, None if gains is None else gains.to(x.dtype))
        ctx.saved = _SavedActivation(x, compressed and x.numel() >= min_elements,
                                     distribution or act_dist, buffer)
        ctx.save_for_backward(gains, rstd)
        return output

    @staticmethod
    def backward(ctx, grad):
        gains, rstd = ctx.saved_tensors
        x = ctx.saved.take()
        ctx.saved = None
        grad_x, grad_gains = rms_norm_backward(grad, x, rstd,
                                               None if gains is None else gains.to(x.dtype))
        if grad_gains is not None:
            grad_gains = grad_gains.to(gains.dtype)
        return grad_x, grad_gains, None, None, None, None


class Relu2Linear(torch.autograd.Function):
    """``linear(relu(z)^2)``; saves ``relu(z)`` and rebuilds the square in
    backward (LCT/components/layers.py:179-222)."""

    @staticmethod
    def forward(ctx, z, weight, bias, buffer=None, compressed=False,
                distribution=None, min_elements=65536):
        relu = z.relu()
        output = F.linear(relu.square(), dense_weight(weight), bias.to(z.dtype))
        ctx.saved = _SavedActivation(relu, compressed and z.numel() >= min_elements,
                                     distribution or act_relu_dist, buffer)
        ctx.save_for_backward(weight)
        ctx.bias_dtype = bias.dtype
        return output

    @staticmethod
    def backward(ctx, grad):
        weight, = ctx.saved_tensors
        relu = ctx.saved.take()
        ctx.saved = None
        g = grad.reshape(-1, grad.shape[-1])
        grad_z = (g @ dense_weight(weight)).reshape(relu.shape)
        grad_z.mul_(2 * relu)
        grad_z.masked_fill_(relu == 0, 0)
        grad_weight = g.T @ relu.square().reshape(-1, relu.shape[-1])
        grad_bias = g.sum(0).to(ctx.bias_dtype)
        return grad_z, grad_weight, grad_bias, None, None, None, None


class _AttentionState:
    """Q, K, V and the attention output between forward and backward.  The
    inputs are BHTD views of contiguous BTHD storage, so each is compressed in
    its storage order (LCT/components/layers.py:225-245)."""

    def __init__(self, tensors, compressed, buffer, distribution):
        self.saved = [_SavedActivation(t.transpose(1, 2) if compressed else t, compressed,
                                       distribution, buffer) for t in tensors]
        self.compressed = compressed

    def unpack(self):
        values = [s.take() for s in self.saved]
        self.saved = []
        return [v.transpose(1, 2) for v in values] if self.compressed else values


def _flash_forward(q, k, v):
    return torch.ops.aten._scaled_dot_product_flash_attention.default(
        q, k, v, 0.0, True, False, scale=ATTENTION_SCALE)


class FlashAttention(torch.autograd.Function):
    """Causal flash attention and the output projection, with the attention's
    inputs and output saved explicitly (LCT/components/layers.py:248-305).
    Inputs are BHTD; the result is BTD."""

    @staticmethod
    def forward(ctx, q, k, v, weight, bias, buffer, compressed, distribution, min_elements):
        out, *auxiliary = _flash_forward(q, k, v)
        hidden = out.transpose(1, 2).reshape(q.shape[0], q.shape[2], -1)
        output = F.linear(hidden, dense_weight(weight), bias.to(out.dtype))
        # lse, cum_seq_q, cum_seq_k, max_q, max_k, philox seed, philox offset;
        # the debug mask (last) is unused.
        ctx.auxiliary = tuple(auxiliary[:7])
        ctx.weight = weight
        ctx.bias_dtype = bias.dtype
        ctx.state = _AttentionState((q, k, v, out), compressed and q.numel() >= min_elements,
                                    buffer, distribution)
        return output

    @staticmethod
    def backward(ctx, grad_output):
        q, k, v, out = ctx.state.unpack()
        batch, heads, length, head_dim = q.shape
        g = grad_output.reshape(-1, grad_output.shape[-1])
        hidden = out.transpose(1, 2).reshape(-1, heads * head_dim)
        grad_weight = g.T @ hidden
        grad_bias = g.sum(0).to(ctx.bias_dtype)
        grad_attention = (g @ dense_weight(ctx.weight)).reshape(
            batch, length, heads, head_dim).transpose(1, 2)
        lse, cum_q, cum_k, max_q, max_k, seed, offset = ctx.auxiliary
        dq, dk, dv = torch.ops.aten._scaled_dot_product_flash_attention_backward.default(
            grad_attention, q, k, v, out, lse, cum_q, cum_k, max_q, max_k,
            0.0, True, seed, offset, scale=ATTENTION_SCALE)
        ctx.state = ctx.auxiliary = ctx.weight = None
        return dq, dk, dv, grad_weight, grad_bias, None, None, None, None


def compress_weight(module, buffer=None, distribution=None):
    """Replace ``module.weight`` by an ``LCTTensor`` (LCT/components/layers.py:308-314).
    Call after initialisation, device placement and checkpoint loading."""
    if isinstance(module.weight, LCTTensor):
        return
    packed = LCTTensor(module.weight, buffer=buffer, dist=distribution or weight_dist)
    del module._parameters["weight"]
    module.weight = packed


class Linear(nn.Linear):
    """Parameter holder of the functional projections: BF16 weight, FP32 bias
    (LCT/components/layers.py:317-326)."""

    def __init__(self, in_features, out_features):
        super().__init__(in_features, out_features, bias=True)
        self.weight = nn.Parameter(self.weight.to(torch.bfloat16))

    def compress_weight(self, buffer=None, distribution=None):
        compress_weight(self, buffer, distribution)


class Embedding(torch.autograd.Function):
    """Embedding lookup from a dense or compressed table
    (LCT/components/layers.py:329-346)."""

    @staticmethod
    def forward(ctx, indices, weight):
        ctx.save_for_backward(indices)
        ctx.num_embeddings = weight.shape[0]
        return F.embedding(indices, dense_weight(weight))

    @staticmethod
    def backward(ctx, grad):
        indices, = ctx.saved_tensors
        return None, torch.ops.aten.embedding_dense_backward(
            grad, indices, ctx.num_embeddings, -1, False)


def named_trainable_tensors(model):
    """``named_parameters`` plus compressed weights, which are not
    ``nn.Parameter``s (LCT/components/layers.py:349-356)."""
    yield from model.named_parameters()
    for name, module in model.named_modules():
        if isinstance(module, (Linear, nn.Embedding)) and isinstance(module.weight, LCTTensor):
            yield (name + "." if name else "") + "weight", module.weight
