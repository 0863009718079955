"""Float64 numpy statement of the decode step's mathematics, written from the
equations (not from the oracle's code), used to pin the oracle's orchestration
of Model::forward (src/model.rs:196-262) and its attention/rope/norm pieces."""
import numpy as np


def rmsnorm(x, w, eps):
    x = np.asarray(x, np.float64)
    return x / np.sqrt(np.mean(x * x) + eps) * np.asarray(w, np.float64)


def rope(x, pos, hd, theta, f32_angle=False):
    """f32_angle: the angle pos*theta^(-2i/hd) is formed in f32 arithmetic (as
    the f32 model computes it) and only sin/cos/rotation are float64."""
    x = np.array(x, np.float64).reshape(-1, hd)
    half = hd // 2
    i = np.arange(half, dtype=np.float64)
    if f32_angle:
        # theta^(-2i/hd) correctly rounded to f32 (numpy's vector powf is not)
        f = (np.float64(np.float32(theta)) ** (-2.0 * i / hd)).astype(np.float32)
        ang = (np.float32(pos) * f).astype(np.float64)
    else:
        ang = pos * theta ** (-2.0 * i / hd)
    c, s = np.cos(ang), np.sin(ang)
    a, b = x[:, :half].copy(), x[:, half:].copy()
    x[:, :half] = a * c - b * s
    x[:, half:] = a * s + b * c
    return x.reshape(-1)


def attention(q, K, V, n_heads, n_kv, hd):
    """q [n_heads*hd]; K, V [ctx][n_kv*hd]."""
    q = np.asarray(q, np.float64).reshape(n_heads, hd)
    K = np.asarray(K, np.float64).reshape(-1, n_kv, hd)
    V = np.asarray(V, np.float64).reshape(-1, n_kv, hd)
    g = n_heads // n_kv
    out = np.empty((n_heads, hd))
    for h in range(n_heads):
        s = K[:, h // g, :] @ q[h] / np.sqrt(hd)
        p = np.exp(s - s.max())
        p /= p.sum()
        out[h] = p @ V[:, h // g, :]
    return out.reshape(-1)


def silu(x):
    x = np.asarray(x, np.float64)
    return x / (1.0 + np.exp(-x))


class Model64:
    """Model::forward in float64 from f32 weights (dict name -> array)."""

    def __init__(self, cfg, W):
        self.cfg, self.W = cfg, W
        self.hd = cfg.head_dim_()
        self.K = [[] for _ in range(cfg.num_hidden_layers)]
        self.V = [[] for _ in range(cfg.num_hidden_layers)]

    def lin(self, name, x):
        y = self.W[name + ".weight"].astype(np.float64) @ x
        b = self.W.get(name + ".bias")
        return y + b if b is not None else y

    def forward(self, token, pos):
        c, W = self.cfg, self.W
        x = W["model.embed_tokens.weight"][token].astype(np.float64)
        for L in range(c.num_hidden_layers):
            p = f"model.layers.{L}."
            xn = rmsnorm(x, W[p + "input_layernorm.weight"], c.rms_norm_eps)
            q = rope(self.lin(p + "self_attn.q_proj", xn), pos, self.hd, c.rope_theta)
            k = rope(self.lin(p + "self_attn.k_proj", xn), pos, self.hd, c.rope_theta)
            v = self.lin(p + "self_attn.v_proj", xn)
            assert len(self.K[L]) == pos
            self.K[L].append(k)
            self.V[L].append(v)
            a = attention(q, np.array(self.K[L]), np.array(self.V[L]), c.num_attention_heads,
                          c.num_key_value_heads, self.hd)
            x = x + self.lin(p + "self_attn.o_proj", a)
            xn = rmsnorm(x, W[p + "post_attention_layernorm.weight"], c.rms_norm_eps)
            inner = silu(self.lin(p + "mlp.gate_proj", xn)) * self.lin(p + "mlp.up_proj", xn)
            x = x + self.lin(p + "mlp.down_proj", inner)
        xn = rmsnorm(x, W["model.norm.weight"], c.rms_norm_eps)
        head = W.get("lm_head.weight", W["model.embed_tokens.weight"])
        return head.astype(np.float64) @ xn
