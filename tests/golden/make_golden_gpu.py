"""Golden vectors of PyTorch's fp32 GPU conv1d + SiLU at BASELINE config 2 (run on the MI355X).

TEST FIXTURE GENERATOR.  BASELINE config 2 defines the packed conv's target as
fp32 ``torch.nn.functional.conv1d`` + SiLU on the GPU, then one bf16 cast.  This
script evaluates exactly that on the config-2 recipe (x [1, 2048, 6144] ~ N(0, 1),
w [6144, 4] ~ N(0, 0.25), bf16, seeds 100 / 101) and keeps, per output element
drawn, its four window values, its four taps, torch's fp32 pre-activation, torch's
fp32 SiLU and the cast bf16 result.  It keeps every element where an fp32 tap sum
in one of four orders differs from torch's pre-activation (the cases that pin how
torch sums), up to ``HARD``, plus ``EASY`` elements drawn uniformly.  A second
draw repeats this with a bias ~ N(0, 1) to pin where the bias is added.

Usage (GPU box): python tests/golden/make_golden_gpu.py OUT.npz
"""
from __future__ import annotations

import sys

import numpy as np
import torch
import torch.nn.functional as F

HARD = 3000
EASY = 1000
T, C, W = 2048, 6144, 4


def bits16(t: torch.Tensor) -> np.ndarray:
    return t.detach().contiguous().cpu().view(torch.int16).numpy().view(np.uint16)


def seeded(shape, seed, scale=1.0):
    g = torch.Generator().manual_seed(seed)
    return (torch.randn(shape, generator=g) * scale).to(torch.bfloat16)


def draw(x, w, bias, rng, tag):
    dev = torch.device("cuda")
    xf, wf = x.to(dev).float(), w.to(dev).float()
    bf = None if bias is None else bias.to(dev).float()
    y = F.conv1d(xf.transpose(1, 2), wf.reshape(C, 1, W), bf, padding=W - 1, groups=C)[..., :T]
    s = F.silu(y)
    out = s.to(torch.bfloat16)
    torch.cuda.synchronize()
    y = y[0].transpose(0, 1).contiguous().cpu().numpy()
    s = s[0].transpose(0, 1).contiguous().cpu().numpy()
    out = bits16(out[0].transpose(0, 1))
    xn = x[0].float().numpy()
    wn = w.float().numpy()
    xpad = np.concatenate([np.zeros((W - 1, C), np.float32), xn])
    P = [(wn[:, j][None, :] * xpad[j:j + T]).astype(np.float32) for j in range(W)]
    orders = [((P[3] + P[0]) + P[1]) + P[2], ((P[0] + P[1]) + P[2]) + P[3],
              ((P[3] + P[2]) + P[1]) + P[0], (P[0] + P[1]) + (P[2] + P[3])]
    if bias is not None:
        orders = [o + bias.float().numpy()[None, :] for o in orders]
    yb = y.view(np.uint32)
    hard = np.zeros((T, C), bool)
    for o in orders:
        hard |= o.view(np.uint32) != yb
    hi = np.flatnonzero(hard.ravel())
    hi = rng.choice(hi, size=min(HARD, hi.size), replace=False)
    ei = rng.choice(np.flatnonzero(~hard.ravel()), size=EASY, replace=False)
    idx = np.sort(np.concatenate([hi, ei]))
    t, c = np.unravel_index(idx, (T, C))
    xb = np.concatenate([np.zeros((W - 1, C), np.uint16), bits16(x[0])])
    win = np.stack([xb[t + j, c] for j in range(W)], axis=1)  # rows t-3 .. t
    res = {f"{tag}_t": t.astype(np.int32), f"{tag}_c": c.astype(np.int32), f"{tag}_x": win,
           f"{tag}_w": bits16(w)[c], f"{tag}_y_f32": yb[t, c], f"{tag}_silu_f32": s.view(np.uint32)[t, c],
           f"{tag}_out": out[t, c], f"{tag}_hard": hard[t, c]}
    if bias is not None:
        res[f"{tag}_bias"] = bits16(bias)[c]
    print(f"{tag}: {int(hard.sum())} elements where some fp32 tap order differs from torch; kept "
          f"{hi.size} of them + {ei.size} others", flush=True)
    return res


def main(path: str) -> None:
    rng = np.random.default_rng(0)
    x = seeded((1, T, C), 100)
    w = seeded((C, W), 101, 0.25)
    out = draw(x, w, None, rng, "conv")
    out.update(draw(x, w, seeded((C,), 102), rng, "bias"))
    np.savez_compressed(path, **out)
    print("wrote", path, flush=True)


if __name__ == "__main__":
    main(sys.argv[1])
