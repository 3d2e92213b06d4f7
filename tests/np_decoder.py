"""Independent float64 numpy formulation of a Whisper text-decoder forward pass.

Written from the architecture (token + positional embedding; per block pre-LN causal
self-attention, pre-LN cross-attention, pre-LN GELU MLP, residuals; final LN; tied logits), not
from the oracle's loop structure: vectorised einsum attention over all positions, exact tanh GELU
evaluated on the f16-rounded input (the reference's table semantics), float64 throughout.  Used
only to check the oracle.
"""

import numpy as np

from whisper4j_amd import synth


def weights64(tensors):
    return {t.name: synth.tensor_to_f32(t).astype(np.float64) for t in tensors}


def _ln(x, g, b, eps=1e-5):
    mu = x.mean(-1, keepdims=True)
    var = ((x - mu) ** 2).mean(-1, keepdims=True)
    return (x - mu) / np.sqrt(var + eps) * g + b


def _gelu_f16(x):
    xh = x.astype(np.float32).astype(np.float16).astype(np.float64)
    return 0.5 * xh * (1.0 + np.tanh(np.sqrt(2.0 / np.pi) * (xh + 0.044715 * xh ** 3)))


def _mha(xq, xkv, W, p, H, causal):
    q = xq @ W[p + "query.weight"].T + W[p + "query.bias"]
    k = xkv @ W[p + "key.weight"].T + W.get(p + "key.bias", 0.0)
    v = xkv @ W[p + "value.weight"].T + W[p + "value.bias"]
    T, d = q.shape
    hd = d // H
    qh = q.reshape(T, H, hd).transpose(1, 0, 2)
    kh = k.reshape(-1, H, hd).transpose(1, 0, 2)
    vh = v.reshape(-1, H, hd).transpose(1, 0, 2)
    s = np.einsum("htd,hsd->hts", qh, kh) / np.sqrt(hd)
    if causal:
        s = s + np.triu(np.full((T, kh.shape[1]), -np.inf), 1)
    s = s - s.max(-1, keepdims=True)
    p_ = np.exp(s)
    p_ /= p_.sum(-1, keepdims=True)
    o = np.einsum("hts,hsd->htd", p_, vh).transpose(1, 0, 2).reshape(T, d)
    return o @ W[p + "out.weight"].T + W[p + "out.bias"]


def forward(W, dims, tokens, xa):
    """Logits [len(tokens)][V] for the full sequence (positions 0..T-1), float64."""
    xa = np.asarray(xa, np.float64)
    x = W["decoder.token_embedding.weight"][tokens] + W["decoder.positional_embedding"][: len(tokens)]
    for i in range(dims.n_text_layer):
        b = f"decoder.blocks.{i}."
        h1 = _ln(x, W[b + "attn_ln.weight"], W[b + "attn_ln.bias"])
        x = x + _mha(h1, h1, W, b + "attn.", dims.n_text_head, True)
        x = x + _mha(_ln(x, W[b + "cross_attn_ln.weight"], W[b + "cross_attn_ln.bias"]), xa, W, b + "cross_attn.",
                     dims.n_text_head, False)
        h = _ln(x, W[b + "mlp_ln.weight"], W[b + "mlp_ln.bias"]) @ W[b + "mlp.0.weight"].T + W[b + "mlp.0.bias"]
        x = x + _gelu_f16(h) @ W[b + "mlp.2.weight"].T + W[b + "mlp.2.bias"]
    x = _ln(x, W["decoder.ln.weight"], W["decoder.ln.bias"])
    return x @ W["decoder.token_embedding.weight"].T
