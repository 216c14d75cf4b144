"""Synthetic draft model for the draft tests: bf16 weights at the trainer's
shapes (src/draft/draft.c:102-114), the safetensors file the loader reads, and
the binary64 weights of the ground truth."""
import json

import numpy as np
import torch

import f64_forward as f64

D, F = 2560, 9728
SHAPES = {"fuse.weight": (D, 2 * D), "wqkv.weight": (6144, D), "wo.weight": (D, 4096),
          "w1.weight": (F, D), "w3.weight": (F, D), "w2.weight": (D, F), "q_norm": (128,),
          "k_norm": (128,), "attn_norm": (D,), "ffn_norm": (D,), "final_norm": (D,)}
# oracle / f64 field name of each tensor
FIELD = {"fuse.weight": "fuse", "wqkv.weight": "wqkv", "wo.weight": "wo", "w1.weight": "w1",
         "w3.weight": "w3", "w2.weight": "w2", "q_norm": "q_norm", "k_norm": "k_norm",
         "attn_norm": "attn_norm", "ffn_norm": "ffn_norm", "final_norm": "final_norm"}


def bf16_bits(a):
    return torch.from_numpy(np.ascontiguousarray(a, np.float32)).to(torch.bfloat16).view(
        torch.int16).numpy().view(np.uint16)


def make_weights(seed):
    """bf16 bits per tensor: matrices N(0, 1/in), norm weights 1 + N(0, 0.1)."""
    r = np.random.default_rng(seed)
    w = {}
    for name, shape in SHAPES.items():
        if len(shape) == 2:
            a = r.standard_normal(shape, dtype=np.float32) / np.float32(np.sqrt(shape[1]))
        else:
            a = 1 + 0.1 * r.standard_normal(shape, dtype=np.float32)
        w[name] = bf16_bits(a)
    return w


def write_safetensors(path, tensors, dtype="BF16", shapes=None):
    """Safetensors layout: u64 LE header length, JSON header, raw data."""
    hdr, off, blobs = {}, 0, []
    for name, a in tensors.items():
        b = np.ascontiguousarray(a).tobytes()
        shape = list((shapes or {}).get(name, a.shape))
        hdr[name] = {"dtype": dtype, "shape": shape, "data_offsets": [off, off + len(b)]}
        off += len(b)
        blobs.append(b)
    hdr["__metadata__"] = {"format": "pt"}
    js = json.dumps(hdr).encode()
    js += b" " * (-len(js) % 8)
    with open(path, "wb") as f:
        f.write(len(js).to_bytes(8, "little"))
        f.write(js)
        for b in blobs:
            f.write(b)


def oracle_arrays(w):
    return {FIELD[n]: np.ascontiguousarray(a) for n, a in w.items()}


def f64_weights(w):
    return {FIELD[n]: f64.bf(a) for n, a in w.items()}
