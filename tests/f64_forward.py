"""Binary64 forward of the slow-AR layer stack: the exact-arithmetic ground
truth for the verify forward (no intermediate bf16 rounding).

The reference-order oracle (or_layer, restating slowar.c:156-260) and the GPU
both round every stage to bf16, each in its own order; this module measures
how far each of them lands from exact arithmetic on the same quantized
weights, caches and inputs, so a test can require the GPU to be no less
accurate than the reference's own order.

Layer math (slowar.c:156-260): x += Wo attn(rope(qk_norm(split(Wqkv rms(x)))));
x += W2 (silu(g) * u) with [g|u] = Wgu rms(x); logits = Whead rms_final(x).
RoPE rotates adjacent pairs (kernels.cu:114-168) with theta 1e6.
"""
import numpy as np

EPS = 1e-6


def bf(bits):
    return (np.ascontiguousarray(bits, np.uint16).astype(np.uint32) << 16).view(
        np.float32).astype(np.float64)


def dequant(w, s, N, K):
    """Exact f64 weights: INT4-g32 packed (low nibble = even k, signed) with
    f16 group scales, or INT8 with f32 row scales."""
    if w.dtype == np.uint8:
        b = w.reshape(N, K // 2)
        lo = ((b << 4).astype(np.int8) >> 4).astype(np.float64)
        hi = (b.astype(np.int8) >> 4).astype(np.float64)
        q = np.empty((N, K), np.float64)
        q[:, 0::2] = lo
        q[:, 1::2] = hi
        sc = s.view(np.float16).astype(np.float64).reshape(N, K // 32)
        return q * np.repeat(sc, 32, axis=1)
    return w.reshape(N, K).astype(np.float64) * s.astype(np.float64)[:, None]


def rms(x, w):
    return x / np.sqrt(np.mean(x * x, axis=-1, keepdims=True) + EPS) * w


def rope(x, pos, heads):
    R = x.shape[0]
    x = x.reshape(R, heads, 64, 2)
    inv = 1e6 ** (-np.arange(64, dtype=np.float64) * 2 / 128)
    ang = np.asarray(pos, np.float64)[:, None] * inv[None, :]
    c, s = np.cos(ang)[:, None, :], np.sin(ang)[:, None, :]
    x0, x1 = x[..., 0], x[..., 1]
    out = np.stack([x0 * c - x1 * s, x1 * c + x0 * s], axis=-1)
    return out.reshape(R, heads * 128)


def layer(W, x, kc, vc, L, pos, vis):
    """W: dict of f64 matrices/vectors; kc, vc: (8, ctx, 128) f64 caches
    updated in place at slots L..L+R-1; vis: per-row ancestor masks."""
    R = x.shape[0]
    qkv = rms(x, W["attn_norm"]) @ W["wqkv"].T
    q, k, v = qkv[:, :4096], qkv[:, 4096:5120], qkv[:, 5120:]
    if W.get("q_norm") is not None:  # the fast-AR layers have no qk-norm
        q = rms(q.reshape(R, 32, 128), W["q_norm"]).reshape(R, 4096)
        k = rms(k.reshape(R, 8, 128), W["k_norm"]).reshape(R, 1024)
    q, k = rope(q, pos, 32), rope(k, pos, 8)
    kc[:, L:L + R] = k.reshape(R, 8, 128).transpose(1, 0, 2)
    vc[:, L:L + R] = v.reshape(R, 8, 128).transpose(1, 0, 2)
    span = L + R
    mask = np.zeros((R, span), bool)
    mask[:, :L] = True
    for r in range(R):
        for b in range(R):
            mask[r, L + b] = bool((int(vis[r]) >> b) & 1)
    att = np.empty((R, 32, 128))
    qh = q.reshape(R, 32, 128)
    for h in range(32):
        sc = qh[:, h] @ kc[h // 4, :span].T / np.sqrt(128.0)
        sc = np.where(mask, sc, -np.inf)
        p = np.exp(sc - sc.max(axis=1, keepdims=True))
        att[:, h] = (p / p.sum(axis=1, keepdims=True)) @ vc[h // 4, :span]
    x = x + att.reshape(R, 4096) @ W["wo"].T
    gu = rms(x, W["ffn_norm"]) @ W["gate_up"].T
    ffn = gu.shape[1] // 2
    g, u = gu[:, :ffn], gu[:, ffn:]
    x = x + (g / (1 + np.exp(-g)) * u) @ W["w2"].T
    return x


def forward(layers, final_norm, head, x_bits, kv_bits, L, parent):
    """layers: list of f64 weight dicts; head: f64 (N, 2560); kv_bits:
    (n_layers, 16, ctx, 128) bf16 bits.  Returns f64 logits (R, N)."""
    R = len(parent)
    depth, vis = [0] * R, []
    for i in range(R):
        if i:
            depth[i] = depth[parent[i]] + 1
        m, j = 0, i
        while j >= 0:
            m |= 1 << j
            j = parent[j]
        vis.append(m)
    pos = [L + d for d in depth]
    x = bf(x_bits)
    for li, W in enumerate(layers):
        kc = bf(kv_bits[li, :8])
        vc = bf(kv_bits[li, 8:])
        x = layer(W, x, kc, vc, L, pos, vis)
    return rms(x, final_norm) @ head.T


def draft_step(W, h, e, kc, vc, pos):
    """Binary64 draft step (src/draft/draft.c:157-202): x = fuse [h; e], one
    backbone-shaped layer at RoPE position / KV slot pos (gate_up = [w1; w3]),
    final RMSNorm.  kc, vc: (8, ctx, 128) f64, updated at slot pos."""
    x = np.concatenate([h, e])[None, :] @ W["fuse"].T
    Wl = dict(W, gate_up=np.vstack([W["w1"], W["w3"]]))
    x = layer(Wl, x, kc, vc, pos, [pos], [1])
    return rms(x, W["final_norm"])[0]


def fastar_step(layers, final_norm, head, hidden, emb_rows, cb):
    """Binary64 logits of fast-AR step cb (src/fastar/fastar.cu:726-789) as
    the uncached causal forward over [hidden, emb_rows[0..cb-1]] at positions
    0..cb (each layer's cache starts empty, depth 11)."""
    x = np.concatenate([bf(hidden)[None], bf(emb_rows[:cb])], axis=0)
    n = cb + 1
    vis = [(1 << (r + 1)) - 1 for r in range(n)]
    for W in layers:
        kc, vc = np.zeros((8, 11, 128)), np.zeros((8, 11, 128))
        x = layer(W, x, kc, vc, 0, list(range(n)), vis)
    return rms(x[-1:], final_norm) @ head.T
