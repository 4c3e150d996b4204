"""A paged-cache backend for Hugging Face transformers models, and an ActKV session on it.

The reference runs models only through a contiguous DynamicCache (actkv/hf/session.py):
- scores come from `output_attentions` on eager attention (session.py:150-156);
- compression is an `index_select` of every layer's keys and values (session.py:195-206).
It names a paged backend that scores with the LSE-recovery kernel as the missing piece
(session.py:12-14; README.md:153, "no model runs on it").  This module is that backend:

  PagedHFCache     a transformers `Cache` over a PagedKVCache for a batch of requests.  A
                   forward's first layer allocates the new tokens' blocks from the host free
                   stack (once per step); every layer's `update` then writes its K/V rows
                   with one actkv_append launch.
  paged_attention_forward
                   the attention function, registered as "actkv_paged": actkv_paged_attention
                   over the layer's paged K/V, causal within the step's new tokens, returning
                   the output and keeping q and the LSE of action tokens for scoring.
  PagedSession     prefill / decode / rounds for a batch of sequences.  Action tokens' q and
                   LSE are kept as they are decoded; `end_round` scores them all in one
                   cal_attn launch (Algorithm 3, each with its causal limit: the cache does not
                   change inside a round, so this equals scoring at every step) and compresses
                   with the device LRFU policy (Algorithm 1) and the paged compaction.

Positions follow the reference's two counters (session.py:4-10): RoPE uses each sequence's
logical position (`seen`), while the paged cache holds the physical tokens; masks are not
built (the kernels apply causality from the cache's lengths).
"""
from __future__ import annotations

import threading

import numpy as np
import torch

from .. import _hip
from ..kernels.lrfu import LRFUConfig, PagedLRFU
from ..kernels.lse_attn import paged_decode_attention
from ..paged import PagedKVCache

try:  # transformers is optional for the rest of the package
    from transformers import AttentionInterface
    from transformers.cache_utils import Cache, CacheLayerMixin
    from transformers.masking_utils import AttentionMaskInterface
except ImportError as e:  # pragma: no cover
    raise ImportError("actkv.hf needs transformers") from e

ATTN_NAME = "actkv_paged"

_tls = threading.local()   # the step being run by this thread's forward pass


class _Step:
    """One forward pass over the batch: n new tokens per request."""

    __slots__ = ("cache", "n", "starts", "plan", "seq", "bt", "kv_len", "capture", "q", "lse", "written",
                 "launch")

    def __init__(self, cache, n, starts, plan, seq, bt, kv_len, capture):
        self.cache, self.n, self.starts, self.plan = cache, n, starts, plan
        self.seq, self.bt, self.kv_len, self.capture = seq, bt, kv_len, capture
        self.q, self.lse = {}, {}
        self.written = 0
        self.launch = None


class _Launch:
    """The step's append and attention launches on a GPU cache.  Everything that is the
    same for every layer (cache strides, the append plan, block tables, the attention
    workspace, the float32 output buffer) is set up once; a layer supplies its index and its
    K/V or query tensors (a decode step runs these for each of the model's layers)."""

    def __init__(self, st, key_states):
        kv = st.cache.kv
        t = kv.kv
        b, hkv, n, d = key_states.shape
        self.lib = _hip.lib()
        self.dev = t.device
        self.stream = _hip.stream(t.device)
        es = t.element_size()
        self.kv_ptr, self.kv_sl_bytes = t.data_ptr(), t.stride(0) * es
        self.kv_code = _hip.dtype_code(t.dtype)
        self.kv_strides = (t.stride(1), t.stride(2), t.stride(3), t.stride(4))
        self.nb, self.bs, self.hkv, self.d = kv.num_blocks, kv.block_size, hkv, d
        self.b, self.n = b, n
        dev_plan, self.r_n, self.mb_plan, self.total = st.plan
        self.plan_ptrs = (dev_plan[2 * self.r_n:].data_ptr(), dev_plan[3 * self.r_n:].data_ptr(),
                          dev_plan.data_ptr(), dev_plan[4 * self.r_n:].data_ptr())
        self.plan_keep = dev_plan
        self.bt, self.seq, self.kv_len = st.bt, st.seq, st.kv_len
        self.out = None

    def append(self, layer, k, v):
        """k, v: [B, n, Hkv, D] contiguous, one dtype -> the cache's layer `layer`."""
        s1, s2, s3, s4 = self.kv_strides
        rc = self.lib.actkv_append(
            self.kv_ptr + layer * self.kv_sl_bytes, self.kv_code, 0, s1, s2, s3, s4, self.nb,
            k.data_ptr(), v.data_ptr(), _hip.dtype_code(k.dtype), 0, self.hkv * self.d, self.d,
            0, self.hkv * self.d, self.d, 1, self.hkv, self.d, self.r_n,
            self.plan_ptrs[0], self.plan_ptrs[1], self.plan_ptrs[2], self.total,
            self.plan_ptrs[3], self.mb_plan, self.mb_plan, self.bs, None, self.stream)
        _hip.check(rc, "actkv_append")

    def attend(self, layer, query, scale, capture):
        """query [B, Hq, n, D] -> (out [B, n, Hq, D] float32, lse [B, n, Hq])."""
        q = query.transpose(1, 2)
        b, n, hq, d = q.shape
        if self.out is None:
            self.hq = hq
            self.out = torch.empty(b, n, hq, d, dtype=torch.float32, device=self.dev)
            self.lse_buf = torch.empty(b, n, hq, dtype=torch.float32, device=self.dev)
            nbytes = int(self.lib.actkv_paged_attention_workspace_size(
                1, b, n, hq, self.hkv, d, self.bt.shape[1], self.bs))
            self.ws = _hip.scratch(self.dev, "attention", nbytes) if nbytes else None
            self.ws_ptr, self.ws_bytes = (self.ws.data_ptr(), self.ws.numel()) if nbytes else (None, 0)
        lse = torch.empty(b, n, hq, dtype=torch.float32, device=self.dev) if capture else self.lse_buf
        out = self.out
        qs = q.stride()
        s1, s2, s3, s4 = self.kv_strides
        rc = self.lib.actkv_paged_attention(
            q.data_ptr(), _hip.dtype_code(q.dtype), 0, qs[0], qs[1], qs[2],
            self.kv_ptr + layer * self.kv_sl_bytes, self.kv_code, 0, s1, s2, s3, s4, self.nb,
            self.bt.data_ptr(), self.bt.stride(0), self.bt.shape[1], self.seq.data_ptr(), None,
            _hip.ptr(self.kv_len), out.data_ptr(), 0, out.stride(0), out.stride(1), out.stride(2),
            lse.data_ptr(), 0, lse.stride(0), lse.stride(1), 1, b, n, hq, self.hkv, d, self.bs,
            float(scale), self.ws_ptr, self.ws_bytes, self.stream)
        _hip.check(rc, "actkv_paged_attention")
        return out, lse


class _PagedLayer(CacheLayerMixin):
    """One model layer's view of the paged cache (writes go through the owner)."""

    is_sliding = False
    is_compileable = False

    def __init__(self, owner: "PagedHFCache", idx: int):
        super().__init__()
        self.owner, self.idx = owner, idx
        self.is_initialized = True

    def lazy_initialization(self, key_states, value_states) -> None:
        pass

    def update(self, key_states, value_states, *args, **kwargs):
        self.owner._write(self.idx, key_states, value_states)
        return key_states, value_states

    def get_mask_sizes(self, query_length: int):
        return self.owner.get_seq_length() + query_length, 0

    def get_seq_length(self) -> int:
        return self.owner.get_seq_length()

    def get_max_length(self) -> int:
        return -1

    def reset(self) -> None:
        raise NotImplementedError("release the requests of the PagedKVCache instead")

    def reorder_cache(self, beam_idx) -> None:
        raise NotImplementedError("beam reordering is not supported by the paged cache")


class PagedHFCache(Cache):
    """transformers Cache over `kv` (a PagedKVCache) for the requests `reqs`, batch row i being
    request reqs[i].  Every layer of the model maps to the same layer of `kv`."""

    def __init__(self, kv: PagedKVCache, reqs):
        self.kv = kv
        self.reqs = list(reqs)
        super().__init__(layers=[_PagedLayer(self, i) for i in range(kv.n_layers)])
        self.step: _Step | None = None
        self.capture = False      # keep q and lse of the next steps (action tokens)
        self.static_step: _Step | None = None  # graph capture: the step's buffers are fixed

    def get_seq_length(self, layer_idx: int = 0) -> int:
        return max((self.kv.seq_used.get(r, 0) for r in self.reqs), default=0)

    def begin_step(self, n: int) -> _Step:
        """Allocate n new tokens per request (host free stack, request order, as n appends)
        and prepare the device side once for all layers."""
        kv = self.kv
        starts = [kv.seq_used.get(r, 0) for r in self.reqs]
        for r, s in zip(self.reqs, starts):
            kv._ensure(r, s + n)
        plan = kv._append_plan(self.reqs, starts, [n] * len(self.reqs))
        for r, s in zip(self.reqs, starts):
            kv.seq_used[r] = s + n
        seq, bt = kv._device_tables(self.reqs)
        kv_len = None
        if n > 1:   # query j of the step sees the prefix and new tokens <= j
            lim = np.asarray(starts, dtype=np.int32)[:, None] + np.arange(1, n + 1, dtype=np.int32)[None, :]
            kv_len = kv._upload(lim.reshape(-1)).view(len(self.reqs), n)
        self.step = _Step(self, n, starts, plan, seq, bt, kv_len, self.capture)
        _tls.step = self.step
        return self.step

    def _write(self, layer: int, key_states: torch.Tensor, value_states: torch.Tensor) -> None:
        b, hkv, n, d = key_states.shape
        if b != len(self.reqs):
            raise ValueError(f"batch of {b} rows, the cache serves {len(self.reqs)} requests")
        st = self.step
        if layer == 0 or st is None or st.written >= self.kv.n_layers:
            if self.static_step is not None:
                # the caller has allocated the step and filled the static buffers
                st = self.step = self.static_step
                st.written = 0
            else:
                st = self.begin_step(n)
        elif st.n != n:
            raise RuntimeError("layers of one forward pass wrote different token counts")
        _tls.step = st
        self._store(layer, st, key_states, value_states)
        st.written += 1

    def _store(self, layer: int, st: "_Step", key_states: torch.Tensor, value_states: torch.Tensor) -> None:
        """The step's new rows of one layer into the paged cache: one actkv_append launch
        (GPU caches only; there is no CPU path)."""
        _hip.require_gpu("PagedHFCache", self.kv.kv)
        b, hkv, n, d = key_states.shape
        # [B, Hkv, n, D] -> [B, n, Hkv, D] contiguous: request r's tokens are rows r*n .. r*n + n - 1
        k = key_states.transpose(1, 2)
        v = value_states.transpose(1, 2)
        k = k if k.is_contiguous() else k.contiguous()
        v = v if v.is_contiguous() else v.contiguous()
        if k.dtype == v.dtype and k.dtype in (torch.float32, torch.float16, torch.bfloat16):
            if st.launch is None:
                st.launch = _Launch(st, key_states)
            st.launch.append(layer, k, v)
        else:   # other source dtypes: the cache's general path converts them first
            self.kv._append_launch(st.plan, k.view(1, b * n, hkv, d), v.view(1, b * n, hkv, d), layer=layer)


def paged_attention_forward(module, query, key, value, attention_mask, scaling=None, dropout=0.0, **kwargs):
    """Attention of `query` [B, Hq, n, D] over the layer's paged K/V (the step's new tokens
    included, causal among them).  Returns ([B, n, Hq, D] in the query dtype, None)."""
    st = getattr(_tls, "step", None)
    if st is None:
        raise RuntimeError("actkv_paged attention runs with a PagedHFCache as past_key_values")
    layer = module.layer_idx
    q = query.transpose(1, 2)                       # [B, n, Hq, D] view, unit last stride
    if st.launch is not None:
        scale = scaling if scaling is not None else query.shape[-1] ** -0.5
        out, lse = st.launch.attend(layer, query, scale, st.capture)
    else:
        out, lse = paged_decode_attention(q, st.cache.kv.kv[layer], st.bt, st.seq, scaling, kv_len=st.kv_len)
    if st.capture:
        st.q[layer], st.lse[layer] = q, lse
    return out.to(query.dtype), None


def _no_mask(*args, **kwargs):
    return None


def register() -> str:
    """Register the attention function (and a no-op mask builder) under "actkv_paged"."""
    AttentionInterface.register(ATTN_NAME, paged_attention_forward)
    AttentionMaskInterface.register(ATTN_NAME, _no_mask)
    return ATTN_NAME


class PagedSession:
    """A batch of sequences served by `model` on a paged cache, compressed with ActKV.

    prefill(ids [B, n], protected)   prompt tokens; protected ones are never evicted
    decode(ids [B], in_action [B])   one token per sequence; action tokens are kept for scoring
    begin_round()                    a new observation-reasoning-action round (Algorithm 1)
    end_round(budget)                score the round's action tokens (one launch over every
                                     layer), update the LRFU keep scores, keep the protected
                                     tokens plus the top `budget`, compact
    Returns logits of each sequence's last position.  Reference: actkv/hf/session.py:91-206
    (prefill, generate, end_round, _compress), with the paged cache instead of DynamicCache."""

    def __init__(self, model, batch: int, max_tokens: int, num_blocks: int | None = None,
                 block_size: int = 16, lrfu: LRFUConfig | None = None, graph: bool = False):
        cfg = model.config
        types = set(getattr(cfg, "layer_types", None) or ["full_attention"])
        if types != {"full_attention"}:
            raise NotImplementedError(f"layer types {sorted(types)}: only full-attention layers are paged")
        p = next(model.parameters())
        dev, dtype = p.device, p.dtype
        _hip.require_gpu("PagedSession", p)
        self.model = model
        self.n_layers = cfg.num_hidden_layers
        self.n_kv = getattr(cfg, "num_key_value_heads", cfg.num_attention_heads)
        self.n_q = cfg.num_attention_heads
        self.head_dim = getattr(cfg, "head_dim", cfg.hidden_size // cfg.num_attention_heads)
        if num_blocks is None:
            num_blocks = batch * (-(-max_tokens // block_size) + 1)
        self.kv = PagedKVCache(num_blocks, block_size, self.n_kv, self.head_dim, n_layers=self.n_layers,
                               dtype=dtype, device=dev)
        self.reqs = list(range(batch))
        self.cache = PagedHFCache(self.kv, self.reqs)
        self.lrfu = PagedLRFU(self.kv, self.reqs, max_tokens, lrfu or LRFUConfig())
        self.seen = [0] * batch           # logical positions (RoPE)
        self.protected = [0] * batch      # protected prefix length
        self.n_action = [0] * batch       # action tokens kept this round
        self._act = []                    # per decode step with action tokens: (q, lse, kv_len, mask)
        self.max_tokens = max_tokens
        self.graph = graph                # decode steps replay a captured HIP graph
        self._g = None                    # the captured step: graph, static buffers, staging
        self._eager_decodes = 0
        model.set_attn_implementation(register())

    # ------------------------------------------------------------------ forward
    @torch.no_grad()
    def _forward(self, ids: torch.Tensor, capture: bool):
        b, n = ids.shape
        dev = self.kv.kv.device
        pos = torch.as_tensor(self.seen, device=dev)[:, None] + torch.arange(n, device=dev)[None, :]
        self.cache.capture = capture
        try:
            out = self.model(input_ids=ids.to(dev), past_key_values=self.cache, position_ids=pos,
                             attention_mask={"full_attention": None}, use_cache=True, logits_to_keep=1)
        finally:
            self.cache.capture = False
        self.seen = [s + n for s in self.seen]
        return out.logits[:, -1]

    def prefill(self, ids: torch.Tensor, protected: bool = False) -> torch.Tensor:
        """ids [B, n] (or [n] for one sequence).  Protected tokens are pinned at the first
        compression (the reference's `protected` prefix, session.py:113-124)."""
        ids = ids.view(len(self.reqs), -1)
        if ids.shape[1] == 0:
            raise ValueError("empty prefill")
        logits = self._forward(ids, capture=False)
        if protected:
            self.protected = [self.kv.seq_used[r] for r in self.reqs]
        return logits

    def begin_round(self) -> None:
        self.lrfu.begin_round()
        self.n_action = [0] * len(self.reqs)
        self._act = []

    # ------------------------------------------------------------------ graph decode
    # A decode step (one token for every sequence) launches a few hundred small kernels; with
    # graph=True it is captured once as a HIP graph and replayed.  What changes between steps
    # lives in fixed device buffers, refreshed by one host-to-device copy before each replay:
    #   meta (int32): positions (int64 as lo/hi) | append plan: source offsets (int64),
    #                 starts, counts, block tables [B, MBG] | lengths [B]
    # The cache's hooks take a static step over these buffers (no allocation or upload while
    # capturing), and the attention's launch shape depends only on the table width MBG.
    def _graph_layout(self):
        b = len(self.reqs)
        mbg = -(-self.max_tokens // self.kv.block_size) + 1
        return b, mbg, 2 * b, 2 * b + 4 * b + b * mbg   # B, MBG, plan offset, lengths offset

    def _graph_fits(self) -> bool:
        _, mbg, _, _ = self._graph_layout()
        bs = self.kv.block_size
        return all(-(-(self.kv.seq_used[r] + 1) // bs) <= mbg for r in self.reqs)

    def _graph_prepare(self, ids: torch.Tensor) -> None:
        """Host side of one graph step: allocate the new tokens' blocks (host free stack, in
        request order), fill the static buffers, advance the lengths."""
        g = self._g
        b, mbg, po, lo = self._graph_layout()
        kv = self.kv
        starts = [kv.seq_used[r] for r in self.reqs]
        for r, s0 in zip(self.reqs, starts):
            kv._ensure(r, s0 + 1)
        k = g["turn"]
        g["turn"] ^= 1
        g["events"][k].synchronize()          # the copy that last read this staging buffer
        host = g["host"][k].numpy()
        host[:po] = np.asarray(self.seen, dtype=np.int64).view(np.int32)
        host[po: po + 2 * b] = np.arange(b, dtype=np.int64).view(np.int32)     # source rows
        host[po + 2 * b: po + 3 * b] = starts
        host[po + 3 * b: po + 4 * b] = 1
        grid = host[po + 4 * b: lo].reshape(b, mbg)
        grid[:] = 0
        for i, r in enumerate(self.reqs):
            t = kv.tables[r]
            grid[i, : len(t)] = t.as_array() if hasattr(t, "as_array") else t
        host[lo: lo + b] = [s0 + 1 for s0 in starts]
        g["meta"].copy_(g["host"][k], non_blocking=True)
        g["events"][k].record()
        g["ids"].copy_(ids.view(b, 1), non_blocking=True)
        for r, s0 in zip(self.reqs, starts):
            kv.seq_used[r] = s0 + 1

    def _graph_capture(self) -> None:
        b, mbg, po, lo = self._graph_layout()
        dev = self.kv.kv.device
        meta = torch.zeros(lo + b, dtype=torch.int32, device=dev)
        plan = (meta[po:lo], b, mbg, b)
        st = _Step(self.cache, 1, None, plan, meta[lo:lo + b], meta[po + 4 * b: lo].view(b, mbg), None, True)
        ids = torch.zeros(b, 1, dtype=torch.long, device=dev)
        pos = meta[:po].view(torch.int64).view(b, 1)
        # the attention workspace exists before the capture (it is cached beyond the graph)
        lib = _hip.lib()
        nbytes = int(lib.actkv_paged_attention_workspace_size(1, b, 1, self.n_q, self.n_kv, self.head_dim, mbg,
                                                              self.kv.block_size))
        if nbytes:
            _hip.scratch(dev, "attention", nbytes)
        torch.cuda.synchronize(dev)
        self.cache.static_step = st
        graph = torch.cuda.CUDAGraph()
        try:
            with torch.cuda.graph(graph):
                logits = self.model(input_ids=ids, past_key_values=self.cache, position_ids=pos,
                                    attention_mask={"full_attention": None}, use_cache=True,
                                    logits_to_keep=1).logits[:, -1]
        finally:
            self.cache.static_step = None
            self.cache.step = None
        host = [torch.empty(lo + b, dtype=torch.int32, pin_memory=True) for _ in range(2)]
        self._g = {"graph": graph, "logits": logits, "step": st, "meta": meta, "ids": ids, "host": host,
                   "events": [torch.cuda.Event() for _ in range(2)], "turn": 0}
        for e in self._g["events"]:
            e.record()

    @torch.no_grad()
    def _graph_decode(self, ids: torch.Tensor) -> torch.Tensor:
        if self._g is None:
            self._graph_capture()
        self._graph_prepare(ids)
        self._g["graph"].replay()
        self.seen = [s + 1 for s in self.seen]
        return self._g["logits"].clone()

    def decode(self, ids: torch.Tensor, in_action=None) -> torch.Tensor:
        """ids [B]: one new token per sequence.  in_action [B] bools (or one bool): which of the
        tokens belong to an action region and are scored at the round's end."""
        b = len(self.reqs)
        flags = [bool(in_action)] * b if in_action is None or isinstance(in_action, bool) else \
            [bool(x) for x in in_action]
        capture = any(flags)
        # graph replay once an eager decode step has run (libraries set up their kernels for
        # the decode shapes on first use, which a capture must not do)
        if self.graph and self._eager_decodes >= 1 and self._graph_fits():
            logits = self._graph_decode(ids)
            st = self._g["step"]
        else:
            logits = self._forward(ids.view(b, 1), capture)
            self._eager_decodes += 1
            st = self.cache.step
        if capture:
            q = torch.stack([st.q[l][:, 0] for l in range(self.n_layers)])          # [L, B, Hq, D]
            lse = torch.stack([st.lse[l][:, 0] for l in range(self.n_layers)])      # [L, B, Hq]
            lim = [self.kv.seq_used[r] for r in self.reqs]
            self._act.append((q, lse, lim, flags))
            self.n_action = [c + int(f) for c, f in zip(self.n_action, flags)]
        return logits

    def _score_round(self) -> None:
        """One cal_attn launch over every layer for the round's action tokens, packed per
        sequence in decode order, each with its causal limit."""
        nmax = max(self.n_action)
        if nmax == 0:
            return
        b, dev = len(self.reqs), self.kv.kv.device
        steps = [[i for i, a in enumerate(self._act) if a[3][j]] for j in range(b)]
        gidx = torch.tensor([s + [s[-1] if s else 0] * (nmax - len(s)) for s in steps], device=dev)  # [B, N]
        qs = torch.stack([a[0] for a in self._act])         # [S, L, B, Hq, D]
        ls = torch.stack([a[1] for a in self._act])         # [S, L, B, Hq]
        rows = torch.arange(b, device=dev)[:, None]
        q = qs[gidx, :, rows].permute(2, 0, 1, 3, 4).contiguous()     # [L, B, N, Hq, D]
        lse = ls[gidx, :, rows].permute(2, 0, 1, 3).contiguous()      # [L, B, N, Hq]
        lim = np.zeros((b, nmax), dtype=np.int32)
        for j, s in enumerate(steps):
            lim[j, : len(s)] = [self._act[i][2][j] for i in s]
        kv_len = _hip.upload_i32(lim, dev).view(b, nmax)
        n_valid = _hip.upload_i32(self.n_action, dev)
        self.kv.cal_attn(self.reqs, q, lse, self.lrfu.scores, self.lrfu.n_seen, layer=None,
                         n_valid=n_valid, kv_len=kv_len)

    def end_round(self, budget) -> list:
        """Algorithm 1 at the end of a round: score, update the keep scores, compress.
        budget: an int or one per sequence (excluding the protected prefix)."""
        self._score_round()
        perms = self.lrfu.evict(budget, protected=self.protected, n_action=self.n_action)
        self._act = []
        return perms
