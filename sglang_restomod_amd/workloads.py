"""Seeded generators for the benchmark workloads: five at head dim 128 (0-4), two at
head dim 256 (5, 6) and two at head dim 512 (7, 8); 9 and 10 are the extend batch of 8 at
head dims 96 and 192 (on the padded tiled extend kernels); 11 and 12 are the verify and
extend batches over an fp8 pool.

Seeding scheme: one CPU ``torch.Generator`` per workload with seed = workload
index. Draw order: lengths, slot permutation, then (on the target device,
with a device generator of the same seed) q, k, v, then scales, then the request
row permutation. The pool has ``sum(seq_len) + 1`` slots; slot 0 is padding, as
in SGLang's token pool. Slots are one global ``randperm`` split across requests,
so every sequence's keys are scattered over the whole pool (page size 1).

The lengths reproduce the example totals quoted for these workloads:
decode-64 sum(ctx) = 295,239; extend-8 sum(P) = 12,453 and sum(E) = 11,179;
fp8 decode-128 sum(ctx) = 2,147,090; verify-32 sum(P + 4) = 254,648.
"""

from __future__ import annotations

from dataclasses import dataclass, field
from typing import Optional

import torch

WORKLOADS = {
    0: dict(name="decode_b1_ctx512_h32kv8_d128_fp16", mode="decode", batch=1, ctx=(512, 512),
            heads=32, heads_kv=8, dim=128, dtype="fp16", kv="fp16"),
    1: dict(name="decode_b64_ctx1k-8k_h64kv8_d128_bf16", mode="decode", batch=64, ctx=(1024, 8192),
            heads=64, heads_kv=8, dim=128, dtype="bf16", kv="bf16"),
    2: dict(name="extend_b8_p0-4k_e256-2k_h40kv8_d128_bf16", mode="extend", batch=8,
            prefix=(0, 4096), extend=(256, 2048), heads=40, heads_kv=8, dim=128, dtype="bf16", kv="bf16"),
    3: dict(name="decode_b128_ctx4k-32k_h32kv8_d128_fp8", mode="decode", batch=128, ctx=(4096, 32768),
            heads=32, heads_kv=8, dim=128, dtype="bf16", kv="fp8"),
    4: dict(name="verify_b32_t4_p2k-16k_h64kv8_d128_bf16", mode="verify", batch=32, prefix=(2048, 16384),
            draft=4, heads=64, heads_kv=8, dim=128, dtype="bf16", kv="bf16"),
    # head dim 256 at a 27B model's two-GPU share (12 query heads, 2 kv heads), the shape
    # of the reference's own D256 kernels
    5: dict(name="decode_b64_ctx1k-8k_h12kv2_d256_bf16", mode="decode", batch=64, ctx=(1024, 8192),
            heads=12, heads_kv=2, dim=256, dtype="bf16", kv="bf16"),
    6: dict(name="extend_b8_p0-4k_e256-2k_h12kv2_d256_bf16", mode="extend", batch=8,
            prefix=(0, 4096), extend=(256, 2048), heads=12, heads_kv=2, dim=256, dtype="bf16", kv="bf16"),
    # head dim 512 (the reference's widest tuned configuration), on the any-head-dim kernel
    7: dict(name="decode_b64_ctx1k-8k_h16kv4_d512_bf16", mode="decode", batch=64, ctx=(1024, 8192),
            heads=16, heads_kv=4, dim=512, dtype="bf16", kv="bf16"),
    8: dict(name="extend_b8_p0-4k_e256-2k_h16kv4_d512_bf16", mode="extend", batch=8,
            prefix=(0, 4096), extend=(256, 2048), heads=16, heads_kv=4, dim=512, dtype="bf16", kv="bf16"),
    9: dict(name="extend_b8_p0-4k_e256-2k_h32kv8_d96_bf16", mode="extend", batch=8,
            prefix=(0, 4096), extend=(256, 2048), heads=32, heads_kv=8, dim=96, dtype="bf16", kv="bf16"),
    10: dict(name="extend_b8_p0-4k_e256-2k_h16kv4_d192_fp16", mode="extend", batch=8,
             prefix=(0, 4096), extend=(256, 2048), heads=16, heads_kv=4, dim=192, dtype="fp16", kv="fp16"),
    11: dict(name="verify_b32_t4_p2k-16k_h64kv8_d128_fp8", mode="verify", batch=32, prefix=(2048, 16384),
             draft=4, heads=64, heads_kv=8, dim=128, dtype="bf16", kv="fp8"),
    # workload 2's extend shape over an fp8 pool (its own seeded lengths, like workload 11)
    12: dict(name="extend_b8_p0-4k_e256-2k_h40kv8_d128_fp8", mode="extend", batch=8,
             prefix=(0, 4096), extend=(256, 2048), heads=40, heads_kv=8, dim=128, dtype="bf16", kv="fp8"),
}

_DT = {"fp16": torch.float16, "bf16": torch.bfloat16}
FP8 = {"e4m3": torch.float8_e4m3fn, "e5m2": torch.float8_e5m2}


@dataclass
class Workload:
    index: int
    name: str
    mode: str
    heads: int
    heads_kv: int
    dim: int
    q: torch.Tensor                 # [T, Hq, D]
    k_pool: torch.Tensor            # [slots, Hkv, D] (fp8 storage for the fp8 workload)
    v_pool: torch.Tensor
    req_to_token: torch.Tensor      # [rows, max_len] int32
    req_pool_indices: torch.Tensor  # [B] int64
    seq_lens: torch.Tensor          # [B] int32 (keys visible to the last query row)
    prefix_lens: torch.Tensor       # [B] int32
    extend_lens: torch.Tensor       # [B] int32 (1 for decode)
    softmax_scale: float
    k_scale: float = 1.0
    v_scale: float = 1.0
    kv_format: Optional[str] = None  # "e4m3" / "e5m2" for fp8 KV
    seq_lens_cpu: list = field(default_factory=list)

    @property
    def batch(self) -> int:
        return int(self.req_pool_indices.numel())

    @property
    def query_start_loc(self) -> torch.Tensor:
        qsl = torch.zeros(self.batch + 1, dtype=torch.int32, device=self.extend_lens.device)
        qsl[1:] = torch.cumsum(self.extend_lens, 0)
        return qsl


def _randint(g, lo, hi, n):
    return torch.randint(lo, hi + 1, (n,), generator=g)


def seq_lengths(index: int) -> list:
    """Keys per sequence of workload ``index`` (the first draws of its generator)."""
    spec = WORKLOADS[index]
    g = torch.Generator().manual_seed(index)
    B = spec["batch"]
    if spec["mode"] == "decode":
        return _randint(g, *spec["ctx"], B).tolist()
    prefix = _randint(g, *spec["prefix"], B)
    ext = _randint(g, *spec["extend"], B) if spec["mode"] == "extend" else torch.full((B,), spec["draft"])
    return (prefix + ext).tolist()


def make(index: int, device="cpu", kv_format: str = "e4m3", batch: Optional[int] = None,
         scale_lens: float = 1.0) -> Workload:
    """Build workload ``index``. ``batch``/``scale_lens`` shrink it for fast tests."""
    spec = WORKLOADS[index]
    g = torch.Generator().manual_seed(index)
    B = spec["batch"]
    if spec["mode"] == "decode":
        ctx = _randint(g, *spec["ctx"], B)
        prefix = ctx - 1
        ext = torch.ones(B, dtype=torch.int64)
    elif spec["mode"] == "extend":
        prefix = _randint(g, *spec["prefix"], B)
        ext = _randint(g, *spec["extend"], B)
        ctx = prefix + ext
    else:
        prefix = _randint(g, *spec["prefix"], B)
        ext = torch.full((B,), spec["draft"], dtype=torch.int64)
        ctx = prefix + ext
    if batch is not None:
        B = min(batch, B)
        ctx, prefix, ext = ctx[:B], prefix[:B], ext[:B]
    if scale_lens != 1.0:
        # shrink while keeping at least one key / one query per sequence
        ext = torch.clamp((ext.double() * scale_lens).round().long(), min=1) if spec["mode"] == "extend" else ext
        prefix = (prefix.double() * scale_lens).round().long()
        if spec["mode"] == "decode":
            prefix = torch.clamp(prefix, min=0)
        ctx = prefix + ext
    total = int(ctx.sum())
    perm = torch.randperm(total, generator=g) + 1  # slot 0 is padding
    max_len = int(ctx.max())
    req_to_token = torch.zeros(B, max_len, dtype=torch.int32)
    off = 0
    for b in range(B):
        n = int(ctx[b])
        req_to_token[b, :n] = perm[off:off + n].to(torch.int32)
        off += n

    dg = torch.Generator(device=device).manual_seed(index)
    H, Hkv, D = spec["heads"], spec["heads_kv"], spec["dim"]
    qdt = _DT[spec["dtype"]]
    T = int(ext.sum())
    slots = total + 1
    q = torch.randn(T, H, D, generator=dg, device=device, dtype=torch.float32).to(qdt)
    k_scale = v_scale = 1.0
    fmt = None
    if spec["kv"] == "fp8":
        fmt = kv_format
        kf = torch.randn(slots, Hkv, D, generator=dg, device=device, dtype=torch.float32)
        vf = torch.randn(slots, Hkv, D, generator=dg, device=device, dtype=torch.float32)
        sc = torch.rand(2, generator=g) * 1.5 + 0.5  # U[0.5, 2.0]
        k_scale, v_scale = float(sc[0]), float(sc[1])
        k_pool = (kf / k_scale).to(FP8[fmt])
        del kf
        v_pool = (vf / v_scale).to(FP8[fmt])
        del vf
    else:
        kvdt = _DT[spec["kv"]]
        k_pool = torch.randn(slots, Hkv, D, generator=dg, device=device, dtype=torch.float32).to(kvdt)
        v_pool = torch.randn(slots, Hkv, D, generator=dg, device=device, dtype=torch.float32).to(kvdt)
    rows = torch.randperm(B, generator=g)
    # request rows live at a permuted position of a larger req_to_token pool
    pool_rows = torch.zeros(B + 1, max_len, dtype=torch.int32)
    pool_rows[rows + 1] = req_to_token
    return Workload(
        index=index, name=spec["name"], mode=spec["mode"], heads=H, heads_kv=Hkv, dim=D,
        q=q, k_pool=k_pool, v_pool=v_pool,
        req_to_token=pool_rows.to(device), req_pool_indices=(rows + 1).to(torch.int64).to(device),
        seq_lens=ctx.to(torch.int32).to(device), prefix_lens=prefix.to(torch.int32).to(device),
        extend_lens=ext.to(torch.int32).to(device), softmax_scale=D ** -0.5,
        k_scale=k_scale, v_scale=v_scale, kv_format=fmt, seq_lens_cpu=[int(x) for x in ctx],
    )


def kv_bytes_per_elem(w: Workload) -> int:
    return w.k_pool.element_size()


def algorithmic_bytes(w: Workload, rows=None) -> int:
    """K+V read once per (token, kv head) + 4 B slot index per token + q in + out, over
    every sequence or over the sequences ``rows``."""
    rows = range(w.batch) if rows is None else rows
    tokens = sum(w.seq_lens_cpu[b] for b in rows)
    ext = w.extend_lens.tolist()
    q_rows = sum(ext[b] for b in rows)
    kv = 2 * tokens * w.heads_kv * w.dim * kv_bytes_per_elem(w)
    idx = 4 * tokens
    qo = 2 * q_rows * w.heads * w.dim * w.q.element_size()
    return kv + idx + qo


def algorithmic_flops(w: Workload, rows=None) -> int:
    """4 * D * Hq * (visible query-key pairs), over every sequence or the sequences ``rows``."""
    pairs = 0
    ext = w.extend_lens.tolist()
    pre = w.prefix_lens.tolist()
    for b in (range(w.batch) if rows is None else rows):
        p, e = pre[b], ext[b]
        # query i (0-based) sees p + i + 1 keys
        pairs += e * p + e * (e + 1) // 2
    return 4 * w.dim * w.heads * pairs
