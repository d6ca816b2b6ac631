"""Write the committed golden vectors for configs 1 and 2.

The expected outputs come from torch's CPU
``torch.nn.functional.scaled_dot_product_attention`` in float64 with autograd
-- a library routine independent of ``oracle/attn_oracle.py`` -- so the oracle
is checked against them rather than against itself.  Inputs are drawn by the
seeded generator the benchmarks use (``np.random.default_rng(config_id)``,
order Q, K, V, dO).  A SHA-256 of every generated input tensor is stored so a
change of numpy's generator is caught instead of silently shifting inputs.

Run from the repository root:  python tests/golden/make_golden.py
"""
from __future__ import annotations

import hashlib
import os
import sys

import numpy as np
import torch

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(os.path.dirname(HERE)))

from oracle.attn_oracle import CONFIGS, seeded_inputs  # noqa: E402  (generator only)


def sha(a: np.ndarray) -> str:
    return hashlib.sha256(np.ascontiguousarray(a).tobytes()).hexdigest()


def torch_attn(q, k, v, do, scale, causal):
    tq = torch.tensor(q, dtype=torch.float64, requires_grad=True)
    tk = torch.tensor(k, dtype=torch.float64, requires_grad=True)
    tv = torch.tensor(v, dtype=torch.float64, requires_grad=True)
    o = torch.nn.functional.scaled_dot_product_attention(tq, tk, tv, is_causal=causal, scale=scale)
    s = (tq @ tk.transpose(-1, -2)) * scale
    if causal:
        L = s.shape[-1]
        s = s.masked_fill(torch.ones(L, L, dtype=torch.bool).triu(1), float("-inf"))
    lse = torch.logsumexp(s, dim=-1)
    res = {"o": o.detach().numpy(), "lse": lse.detach().numpy()}
    if do is not None:
        o.backward(torch.tensor(do, dtype=torch.float64))
        res.update(dq=tq.grad.numpy(), dk=tk.grad.numpy(), dv=tv.grad.numpy())
    return res


def main():
    # Config 1: full inputs and outputs (tiny).
    c1 = CONFIGS[1]
    x = seeded_inputs(c1)
    r = torch_attn(x["q"], x["k"], x["v"], None, c1.scale, c1.causal)
    np.savez_compressed(
        os.path.join(HERE, "c1_fwd.npz"),
        q=x["q"], k=x["k"], v=x["v"],
        o=r["o"].astype(np.float64), lse=r["lse"].astype(np.float64),
        scale=np.float64(c1.scale),
        sha_q=sha(x["q"]), sha_k=sha(x["k"]), sha_v=sha(x["v"]),
    )
    # Config 2: outputs for two heads (float32 storage), input hashes, and
    # float64 checksums of the full output tensors.
    c2 = CONFIGS[2]
    x = seeded_inputs(c2)
    r = torch_attn(x["q"], x["k"], x["v"], x["do"], c2.scale, c2.causal)
    heads = np.array([[0, 0], [7, 7]], dtype=np.int64)
    out = dict(heads=heads, scale=np.float64(c2.scale))
    for n in ("q", "k", "v", "do"):
        out["sha_" + n] = sha(x[n])
    for n in ("o", "lse", "dq", "dk", "dv"):
        out[n + "_heads"] = np.stack([r[n][b, h] for b, h in heads]).astype(np.float32)
        out[n + "_sum"] = np.float64(r[n].sum())
        out[n + "_abssum"] = np.float64(np.abs(r[n]).sum())
    np.savez_compressed(os.path.join(HERE, "c2_fwdbwd.npz"), **out)
    print("wrote c1_fwd.npz and c2_fwdbwd.npz")


if __name__ == "__main__":
    main()
