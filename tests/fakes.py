"""Engine fakes for the backend tests: exactly the fields the backend reads from
SGLang's model runner, forward batch, layer and KV pool
(sglang_restomod/attention/v100/flash_attn_v100_backend.py:183-226, 332-380,
567-621, 975-1000, 1174-1191), with the token pool's write semantics
(quantize as ``(x / scale).to(fp8)``, stored as bytes and viewed back).
"""

from __future__ import annotations

from dataclasses import dataclass, field
from types import SimpleNamespace
from typing import Optional

import torch

FP8 = (torch.float8_e4m3fn, torch.float8_e5m2)


class ForwardMode:
    def __init__(self, name: str):
        self.name = name

    def is_decode(self):
        return self.name == "DECODE"

    def is_idle(self):
        return self.name == "IDLE"

    def is_decode_or_idle(self):
        return self.name in ("DECODE", "IDLE")

    def is_extend(self):
        return self.name in ("EXTEND", "MIXED", "TARGET_VERIFY", "DRAFT_EXTEND", "DRAFT_EXTEND_V2")

    def is_target_verify(self):
        return self.name == "TARGET_VERIFY"

    def is_draft_extend_v2(self):
        return self.name == "DRAFT_EXTEND_V2"

    def is_draft_extend(self, include_v2: bool = False):
        return self.name == "DRAFT_EXTEND" or (include_v2 and self.name == "DRAFT_EXTEND_V2")


class SpecAlgorithm:
    def __init__(self, kind: str = "NONE"):
        self.kind = kind

    def is_speculative(self):
        return self.kind != "NONE"

    def is_eagle(self):
        return self.kind in ("EAGLE", "EAGLE3")

    def is_dflash_family(self):
        return self.kind == "DFLASH"


class TokenToKVPool:
    """Flat per-layer pools [size + 1, Hkv, D]; slot 0 is the padding slot."""

    def __init__(self, size, dtype, head_num, head_dim, layer_num, device, swa_map=None):
        self.size = size
        self.dtype = dtype
        self.store_dtype = torch.uint8 if dtype in FP8 else dtype
        self.k_buffer = [torch.zeros(size + 1, head_num, head_dim, dtype=self.store_dtype, device=device)
                         for _ in range(layer_num)]
        self.v_buffer = [torch.zeros_like(b) for b in self.k_buffer]
        self.writes = 0
        if swa_map is not None:
            self.full_to_swa_index_mapping = swa_map

    def _view(self, buf):
        return buf.view(self.dtype) if self.store_dtype != self.dtype else buf

    def get_key_buffer(self, layer_id):
        return self._view(self.k_buffer[layer_id])

    def get_value_buffer(self, layer_id):
        return self._view(self.v_buffer[layer_id])

    def get_kv_buffer(self, layer_id):
        return self.get_key_buffer(layer_id), self.get_value_buffer(layer_id)

    def set_kv_buffer(self, layer, loc, cache_k, cache_v, k_scale=None, v_scale=None):
        self.writes += 1
        if getattr(self, "full_to_swa_index_mapping", None) is not None and \
                getattr(layer, "sliding_window_size", -1) is not None and getattr(layer, "sliding_window_size", -1) >= 0:
            # an SWA pool stores its sliding-window layers at their SWA slots
            loc = self.full_to_swa_index_mapping[loc]
        if cache_k.dtype != self.dtype:
            if k_scale is not None:
                cache_k = cache_k / k_scale
            if v_scale is not None:
                cache_v = cache_v / v_scale
            cache_k = cache_k.to(self.dtype)
            cache_v = cache_v.to(self.dtype)
        if self.store_dtype != self.dtype:
            cache_k = cache_k.view(self.store_dtype)
            cache_v = cache_v.view(self.store_dtype)
        self.k_buffer[layer.layer_id][loc] = cache_k
        self.v_buffer[layer.layer_id][loc] = cache_v

    def translate_loc_from_full_to_swa(self, loc):
        return self.full_to_swa_index_mapping[loc]


@dataclass
class Layer:
    tp_q_head_num: int
    tp_k_head_num: int
    head_dim: int = 128
    layer_id: int = 0
    scaling: float = 128 ** -0.5
    k_scale: Optional[torch.Tensor] = None
    v_scale: Optional[torch.Tensor] = None
    k_scale_float: float = 1.0
    v_scale_float: float = 1.0
    sliding_window_size: int = -1
    is_cross_attention: bool = False
    attn_type: object = field(default_factory=lambda: SimpleNamespace(name="DECODER"))
    logit_cap: float = 0.0
    xai_temperature_len: int = -1

    @property
    def qk_head_dim(self):
        return self.head_dim

    @property
    def v_head_dim(self):
        return self.head_dim


class Engine:
    """A model runner plus a slot allocator over a shuffled token pool.

    At ``page_size`` 1 every token takes a random free slot. At a larger page size the
    pool is cut into pages of ``page_size`` consecutive slots, handed out in random order,
    and position ``p`` of a request lives at offset ``p % page_size`` of the request's page
    ``p // page_size`` (SGLang's paged allocator); ``req_to_token`` still holds one slot
    per token. Page 0 holds the padding slot 0 and is never handed out.
    """

    def __init__(self, device, *, hq=8, hkv=2, head_dim=128, kv_dtype=torch.bfloat16, pool_size=4096,
                 max_reqs=16, context_len=2048, layers=1, spec="NONE", topk=1, draft_worker=False,
                 seed=0, swa=False, page_size=1):
        self.device = torch.device(device)
        g = torch.Generator().manual_seed(seed)
        self.gen = g
        self.page_size = int(page_size)
        if self.page_size > 1:
            if pool_size % self.page_size:
                raise ValueError("pool_size must be a multiple of page_size")
            pages = pool_size // self.page_size
            # pages 1 .. pages-1 (page 0 would hold the padding slot)
            self.free_pages = (torch.randperm(pages - 1, generator=g) + 1).tolist()
            self.free = []
        else:
            self.free = (torch.randperm(pool_size, generator=g) + 1).tolist()
        swa_map = None
        if swa:
            # a second numbering of the same slots (the SWA pool of a hybrid model)
            swa_map = torch.zeros(pool_size + 1, dtype=torch.int64)
            swa_map[1:] = torch.randperm(pool_size, generator=g) + 1
            swa_map = swa_map.to(self.device)
        self.pool = TokenToKVPool(pool_size, kv_dtype, hkv, head_dim, layers, self.device, swa_map)
        req_to_token = torch.zeros(max_reqs, context_len, dtype=torch.int32, device=self.device)
        self.lens = [0] * max_reqs
        self.runner = SimpleNamespace(
            device=str(self.device),
            page_size=self.page_size,
            model_config=SimpleNamespace(context_len=context_len, head_dim=head_dim, v_head_dim=head_dim),
            req_to_token_pool=SimpleNamespace(req_to_token=req_to_token, size=max_reqs),
            token_to_kv_pool=self.pool,
            kv_cache_dtype=kv_dtype,
            spec_algorithm=SpecAlgorithm(spec),
            is_draft_worker=draft_worker,
            server_args=SimpleNamespace(speculative_eagle_topk=topk),
        )

    @property
    def req_to_token(self):
        return self.runner.req_to_token_pool.req_to_token

    def alloc(self, row: int, n: int) -> torch.Tensor:
        """Give request ``row`` n more tokens; returns their slots (the out_cache_loc)."""
        start = self.lens[row]
        if self.page_size > 1:
            ps = self.page_size
            got = []
            for pos in range(start, start + n):
                if pos % ps == 0:
                    page = self.free_pages.pop()
                else:  # the page of the previous position
                    prev = got[-1] if got else int(self.req_to_token[row, pos - 1])
                    page = prev // ps
                got.append(page * ps + pos % ps)
            slots = torch.tensor(got, dtype=torch.int64)
        else:
            slots = torch.tensor([self.free.pop() for _ in range(n)], dtype=torch.int64)
        self.req_to_token[row, start:start + n] = slots.to(self.device, torch.int32)
        self.lens[row] += n
        return slots.to(self.device)

    def fill(self, layer_id: int, slots: torch.Tensor, k: torch.Tensor, v: torch.Tensor, layer=None):
        """Write K/V for cached positions (the prefix a real engine computed earlier)."""
        lay = layer or SimpleNamespace(layer_id=layer_id)
        self.pool.set_kv_buffer(lay, slots, k, v, getattr(lay, "k_scale", None), getattr(lay, "v_scale", None))

    def batch(self, mode: str, rows, *, new_tokens, prefix_lens=None, draft_token_num=None):
        """A ForwardBatch for ``rows`` after allocating ``new_tokens[i]`` tokens each.

        For TARGET_VERIFY, seq_lens are the lengths before the draft tokens (as the
        engine hands them), and the draft tokens' slots are allocated here.
        """
        rows = list(rows)
        before = [self.lens[r] for r in rows]
        locs = [self.alloc(r, n) for r, n in zip(rows, new_tokens)]
        dev = self.device
        seq_after = [self.lens[r] for r in rows]
        fb = SimpleNamespace(
            forward_mode=ForwardMode(mode),
            batch_size=len(rows),
            req_pool_indices=torch.tensor(rows, dtype=torch.int64, device=dev),
            out_cache_loc=torch.cat(locs) if locs else torch.zeros(0, dtype=torch.int64, device=dev),
            spec_info=None,
            encoder_lens=None,
        )
        if mode == "TARGET_VERIFY":
            fb.seq_lens = torch.tensor(before, dtype=torch.int64, device=dev)
            fb.seq_lens_cpu = torch.tensor(before, dtype=torch.int64)
            fb.spec_info = SimpleNamespace(draft_token_num=int(draft_token_num))
        else:
            fb.seq_lens = torch.tensor(seq_after, dtype=torch.int64, device=dev)
            fb.seq_lens_cpu = torch.tensor(seq_after, dtype=torch.int64)
        if mode != "DECODE":
            pre = before if prefix_lens is None else prefix_lens
            fb.extend_prefix_lens = torch.tensor(pre, dtype=torch.int32, device=dev)
            fb.extend_seq_lens = torch.tensor(new_tokens, dtype=torch.int32, device=dev)
            fb.extend_seq_lens_cpu = list(new_tokens)
        fb.seq_lens_sum = int(sum(fb.seq_lens_cpu.tolist()))
        fb.input_ids = torch.zeros(sum(new_tokens), dtype=torch.int64, device=dev)
        fb.before = before
        return fb
