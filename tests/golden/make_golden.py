"""Write the golden attention fixtures (tests/golden/*.npz).

    python tests/golden/make_golden.py

Each fixture is one tiny paged-attention case over a token pool with shuffled
slots. Inputs are stored bit-exact in their storage dtype (bf16 / fp16 as uint16
bits, fp8 as bytes). The expected output (float64) comes from the scalar loops
of ``oracle.attention.brute_force``, one (sequence, q head) at a time, with the
visibility rule written out here:

    key j of sequence b is visible to its query row i when
        j < seq_len[b],
        j <= prefix[b] + i           (causal),
        j >= prefix[b] + i - window  (window >= 0).

Scores use softmax_scale * k_scale and outputs are multiplied by v_scale
(sglang_restomod/attention/v100/tilelang/_paged_adapter.py:658, 753-754).
fp8 bytes are dequantized with torch's cast (the reference's table,
_paged_adapter.py:373-386). The fixtures are data only: inputs and outputs.
"""

from __future__ import annotations

import os
import sys

import numpy as np
import torch

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(os.path.dirname(HERE)))

from oracle.attention import brute_force  # noqa: E402

D = 128
CASES = {
    # name: (q dtype, kv dtype, Hq, Hkv, prefix, extend, causal, window, k_scale, v_scale[, seq_lens])
    # seq_lens defaults to prefix + extend; decode_empty_row gives sequence 0 no key at all
    "decode_bf16": ("bf16", "bf16", 8, 2, [4, 0, 36], [1, 1, 1], True, -1, 1.0, 1.0),
    "decode_fp16_gqa5": ("fp16", "fp16", 10, 2, [9, 22], [1, 1], True, -1, 1.0, 1.0),
    "decode_empty_row": ("bf16", "bf16", 4, 1, [-1, 7], [1, 1], True, -1, 1.0, 1.0, [0, 8]),
    "decode_window": ("bf16", "bf16", 8, 2, [30, 5], [1, 1], True, 6, 1.0, 1.0),
    "decode_e4m3": ("bf16", "e4m3", 8, 2, [17, 33], [1, 1], True, -1, 1.5, 0.5),
    "decode_e5m2": ("fp16", "e5m2", 8, 2, [17, 33], [1, 1], True, -1, 0.75, 2.0),
    "extend_bf16": ("bf16", "bf16", 8, 2, [3, 0], [4, 6], True, -1, 1.0, 1.0),
    "extend_noncausal_window": ("bf16", "bf16", 6, 3, [5, 2], [3, 4], False, 2, 1.0, 1.0),
    "extend_e4m3": ("bf16", "e4m3", 4, 1, [8, 0], [5, 3], True, -1, 1.25, 0.8),
    "verify_fp16": ("fp16", "fp16", 8, 1, [20, 9], [3, 3], True, -1, 1.0, 1.0),
    "verify_e5m2": ("bf16", "e5m2", 8, 2, [12, 25], [4, 4], True, -1, 0.5, 1.5),
}
TORCH = {"bf16": torch.bfloat16, "fp16": torch.float16, "e4m3": torch.float8_e4m3fn, "e5m2": torch.float8_e5m2}


def _store(t: torch.Tensor) -> np.ndarray:
    if t.dtype in (torch.bfloat16, torch.float16):
        return t.view(torch.int16).numpy().view(np.uint16)
    return t.view(torch.uint8).numpy()


def make(name, spec, seed):
    qdt, kvdt, hq, hkv, prefix, extend, causal, window, ks, vs = spec[:10]
    g = torch.Generator().manual_seed(seed)
    B = len(prefix)
    seq = list(spec[10]) if len(spec) > 10 else [p + e for p, e in zip(prefix, extend)]
    slots_total = sum(seq) + 1
    perm = (torch.randperm(slots_total - 1, generator=g) + 1).tolist()
    width = max(max(seq), 1) + 3
    rows = B + 2
    r2t = np.zeros((rows, width), dtype=np.int32)
    rpi = (torch.randperm(rows, generator=g)[:B]).numpy().astype(np.int64)
    pos = 0
    for b in range(B):
        r2t[rpi[b], :seq[b]] = perm[pos:pos + seq[b]]
        pos += seq[b]
    T = sum(extend)
    q = torch.randn(T, hq, D, generator=g).to(TORCH[qdt])
    k = torch.randn(slots_total, hkv, D, generator=g)
    v = torch.randn(slots_total, hkv, D, generator=g)
    if kvdt in ("e4m3", "e5m2"):
        k = (k / ks).to(TORCH[kvdt])
        v = (v / vs).to(TORCH[kvdt])
    else:
        k, v = k.to(TORCH[kvdt]), v.to(TORCH[kvdt])
    qf, kf, vf = q.double().numpy(), k.double().numpy(), v.double().numpy()
    qsl = np.zeros(B + 1, dtype=np.int32)
    qsl[1:] = np.cumsum(extend)
    G = hq // hkv
    scale = D ** -0.5
    out = np.zeros((T, hq, D))
    for b in range(B):
        n, P, E = seq[b], prefix[b], extend[b]
        if E == 0:
            continue
        sl = r2t[rpi[b], :n].astype(np.int64)
        vis = np.zeros((E, n), dtype=bool)
        for i in range(E):
            for j in range(n):
                ok = j < n
                if causal:
                    ok = ok and j <= P + i
                if window >= 0:
                    ok = ok and j >= P + i - window
                vis[i, j] = ok
        for h in range(hq):
            kv = h // G
            qr = qf[qsl[b]:qsl[b + 1], h, :]
            out[qsl[b]:qsl[b + 1], h, :] = brute_force(qr, kf[sl, kv, :], vf[sl, kv, :], scale * ks, vis) * vs
    np.savez_compressed(
        os.path.join(HERE, name + ".npz"),
        q=_store(q), q_dtype=qdt, k=_store(k), v=_store(v), kv_dtype=kvdt,
        req_to_token=r2t, req_pool_indices=rpi, seq_lens=np.array(seq, dtype=np.int32),
        prefix_lens=np.array([max(p, 0) for p in prefix], dtype=np.int32), query_start_loc=qsl,
        causal=np.int32(causal), window=np.int32(window), softmax_scale=np.float64(scale),
        k_scale=np.float64(ks), v_scale=np.float64(vs), expected=out,
    )


if __name__ == "__main__":
    for i, (name, spec) in enumerate(sorted(CASES.items())):
        make(name, spec, 1000 + i)
        print("wrote", name)
