"""An independent float64 formulation of the Whisper audio encoder (numpy, written from the model's
definition rather than from the oracle's loops): Conv1d as a sum of three shifted matrix products,
GELU as the tanh form evaluated at the input's f16 value (the reference's table definition,
main/tensor/Tensor.java:493-501), softmax attention per head, pre-LN blocks, ln_post.  Test
infrastructure: it pins the oracle's encoder to within float32 rounding."""

import numpy as np

from whisper4j_amd import synth


def _gelu(x):
    h = x.astype(np.float32).astype(np.float16).astype(np.float64)
    return 0.5 * h * (1.0 + np.tanh(np.sqrt(2.0 / np.pi) * (h + 0.044715 * h ** 3)))


def _ln(x, g, b):
    m = x.mean(-1, keepdims=True)
    v = ((x - m) ** 2).mean(-1, keepdims=True)
    return (x - m) / np.sqrt(v + 1e-5) * g + b


def _conv(x, w, b, stride):
    """x [len][in] time-major, w [out][in][3], padding 1 -> [out_len][out]."""
    n = x.shape[0]
    xp = np.concatenate([np.zeros((1, x.shape[1])), x, np.zeros((1, x.shape[1]))])
    out_len = (n + 2 - 3) // stride + 1
    y = np.zeros((out_len, w.shape[0]))
    for k in range(3):
        y += xp[k: k + stride * (out_len - 1) + 1: stride] @ w[:, :, k].T
    return y + b


def encoder_forward(edims, tensors, mel):
    t = {x.name: synth.tensor_to_f32(x).astype(np.float64) for x in tensors}
    d, H = edims.n_audio_state, edims.n_audio_head
    x = _gelu(_conv(mel.T.astype(np.float64), t["encoder.conv1.weight"], t["encoder.conv1.bias"].ravel(), 1))
    x = _gelu(_conv(x, t["encoder.conv2.weight"], t["encoder.conv2.bias"].ravel(), 2))
    x = x + t["encoder.positional_embedding"]
    T = x.shape[0]
    for i in range(edims.n_audio_layer):
        p = f"encoder.blocks.{i}."
        h = _ln(x, t[p + "attn_ln.weight"], t[p + "attn_ln.bias"])
        q = h @ t[p + "attn.query.weight"].T + t[p + "attn.query.bias"]
        k = h @ t[p + "attn.key.weight"].T
        v = h @ t[p + "attn.value.weight"].T + t[p + "attn.value.bias"]
        q, k, v = (a.reshape(T, H, 64).transpose(1, 0, 2) for a in (q, k, v))
        s = q @ k.transpose(0, 2, 1) / 8.0
        s = np.exp(s - s.max(-1, keepdims=True))
        s /= s.sum(-1, keepdims=True)
        o = (s @ v).transpose(1, 0, 2).reshape(T, d)
        x = x + o @ t[p + "attn.out.weight"].T + t[p + "attn.out.bias"]
        h = _ln(x, t[p + "mlp_ln.weight"], t[p + "mlp_ln.bias"])
        h = _gelu(h @ t[p + "mlp.0.weight"].T + t[p + "mlp.0.bias"])
        x = x + h @ t[p + "mlp.2.weight"].T + t[p + "mlp.2.bias"]
    return _ln(x, t["encoder.ln_post.weight"], t["encoder.ln_post.bias"])
