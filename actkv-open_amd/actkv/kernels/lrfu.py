"""Device LRFU keep score (ActKV Algorithm 1) for the paged cache.

The reference keeps, per layer and cached token, the running mean `act` of the attention the
current round's action tokens paid to the token, and a keep score updated once per compression
step: ks = decay * ks + act * hit, hit = the token is in the top-p mass of act
(actkv/eviction.py:145-224, nucleus actkv/eviction.py:36-50).  The paged cache compacts whole
slots (all layers together), so its keep set is the protected prefix plus the top-`budget`
tokens by the layer-average of ks; the compaction permutation then permutes ks.

Here `act` is the cal_attn output of the round (running mean over the action queries of the
GQA-group max, per KV head), reduced over KV heads inside the kernel.
"""
from __future__ import annotations

from dataclasses import dataclass

import torch

from .. import _hip
from .compaction import upload_i32

_REDUCE = {"mean": _hip.REDUCE_MEAN, "max": _hip.REDUCE_MAX}


def _per_request(v, n):
    return [int(x) for x in v] if isinstance(v, (list, tuple)) else [int(v)] * n


def lrfu_update(scores: torch.Tensor, ks: torch.Tensor, seq_used, protected=0, active=True,
                decay: float = 0.5, top_p: float = 0.9, head_reduce: str = "mean",
                return_hits: bool = False):
    """ks[l, r, t] <- decay * ks + act * hit over t in [protected[r], seq_used[r]) for every
    layer l and request r (eviction.py:209-218), act = head reduction of scores[l, r, :, t].

    scores: float32 [L, R, Hkv, W] on the GPU (the round's action-region scores); ks: float32
    [L, R, W2] on the GPU, updated in place.  seq_used / protected / active: one value for
    every request or a list.  Returns the hit mask [L, R, max(seq_used)] bool when
    return_hits (entries below protected[r] or past seq_used[r] are undefined).
    protected may instead be a bool tensor [R, >=max(seq_used)] of pinned tokens (the paged
    cache's `pinned` masks): pinned tokens are left out of the nucleus and keep their ks."""
    if head_reduce not in _REDUCE:
        raise ValueError(head_reduce)
    dev = _hip.require_gpu("lrfu_update", scores, ks)
    if scores.dim() != 4 or ks.dim() != 3:
        raise ValueError(f"scores must be [L, R, Hkv, W] and ks [L, R, W], got {tuple(scores.shape)}, {tuple(ks.shape)}")
    L, R, H, W = scores.shape
    if ks.shape[0] != L or ks.shape[1] != R:
        raise ValueError(f"ks {tuple(ks.shape)} does not match scores {tuple(scores.shape)}")
    if scores.dtype != torch.float32 or ks.dtype != torch.float32:
        raise ValueError("scores and ks are float32")
    if scores.stride(-1) != 1 or ks.stride(-1) != 1:
        raise ValueError("scores and ks need a unit stride in their last dimension")
    seqs = _per_request(seq_used, R)
    pmask = None
    if isinstance(protected, torch.Tensor):
        pmask = protected.to(device=dev, dtype=torch.bool)
        if pmask.dim() != 2 or pmask.shape[0] != R or pmask.shape[1] < max(seqs, default=0):
            raise ValueError(f"a pinned mask must be [R, >=seq_used], got {tuple(protected.shape)}")
        if pmask.stride(-1) != 1:
            pmask = pmask.contiguous()
        prots = [0] * R
    else:
        prots = _per_request(protected, R)
    acts = [1 if a else 0 for a in (active if isinstance(active, (list, tuple)) else [active] * R)]
    max_seq = max(seqs) if seqs else 0
    if max_seq > W or max_seq > ks.shape[2]:
        raise ValueError(f"seq_used {max_seq} exceeds the scores ({W}) or ks ({ks.shape[2]}) width")
    params = upload_i32(seqs + prots + acts, dev)
    hits = torch.empty(L, R, max(max_seq, 1), dtype=torch.bool, device=dev) if return_hits else None
    _lrfu_launch(scores, ks, params[:R], None if pmask is not None else params[R:2 * R], pmask,
                 params[2 * R:], max_seq, decay, top_p, head_reduce, hits)
    return hits


def _lrfu_launch(scores, ks, seq_dev, prot_count_dev, pmask, active_dev, max_seq, decay, top_p,
                 head_reduce, hits=None):
    """actkv_lrfu_update with device-side per-request parameters (int32 tensors)."""
    dev = scores.device
    L, R, H, _ = scores.shape
    nbytes = int(_hip.lib().actkv_lrfu_workspace_size(L, R, max_seq))
    ws = _hip.scratch(dev, "lrfu", nbytes)
    rc = _hip.lib().actkv_lrfu_update(
        scores.data_ptr(), scores.stride(0), scores.stride(1), scores.stride(2), L, H, R,
        seq_dev.data_ptr(), _hip.ptr(prot_count_dev),
        _hip.ptr(pmask), 0 if pmask is None else pmask.stride(0), _hip.ptr(active_dev),
        ks.data_ptr(), ks.stride(0), ks.stride(1),
        _hip.ptr(hits), 0 if hits is None else hits.stride(0), 0 if hits is None else hits.stride(1),
        float(decay), float(top_p), _REDUCE[head_reduce], max_seq, ws.data_ptr(), ws.numel(),
        _hip.stream(dev))
    _hip.check(rc, "actkv_lrfu_update")


@dataclass
class LRFUConfig:
    """Algorithm 1 hyperparameters (actkv/config.py:9-17 defaults)."""
    decay: float = 0.5
    top_p: float = 0.90
    head_reduce: str = "mean"


class PagedLRFU:
    """ActionLRFU (eviction.py:145-224) on a PagedKVCache for a fixed batch of requests.

    Per round: begin_round() clears the action-region scores; the caller scores the round's
    action tokens with cache.cal_attn(..., out=self.scores, n_seen=self.n_seen); evict()
    then updates the keep scores (a request with no action tokens this round only decays),
    keeps the protected tokens plus the top-`budget` tokens by the layer-average keep score,
    compacts the cache, and moves the keep scores and pins with their tokens.  The batch's
    keep scores and pins live in device matrices [L, R, W] / [R, W], so a round is a fixed
    handful of launches whatever the batch size."""

    def __init__(self, cache, reqs, max_tokens: int, cfg: LRFUConfig | None = None):
        self.cache, self.reqs = cache, list(reqs)
        self.cfg = cfg or LRFUConfig()
        dev = cache.kv.device
        L, R, H = cache.n_layers, len(self.reqs), cache.n_kv_heads
        self.max_tokens = max_tokens
        # per-token buffers span whole blocks: cal_attn writes every slot of a request's last
        # block, so its output must be as wide as the block table covers (lse_attn.py:139-142)
        width = -(-max_tokens // cache.block_size) * cache.block_size
        self.width = width
        self.ks = torch.zeros(L, R, width, dtype=torch.float32, device=dev)
        self._ks_alt = torch.zeros_like(self.ks)
        self.scores = torch.zeros(L, R, H, width, dtype=torch.float32, device=dev)
        self.n_seen = torch.zeros(R, dtype=torch.int32, device=dev)
        self.pins = torch.zeros(R, width, dtype=torch.bool, device=dev)
        self._pins_alt = torch.zeros_like(self.pins)
        self.pin_counts = None           # host counts once the batch has been evicted

    def begin_round(self) -> None:
        """Action-region state is reset on entry to each action region (eviction.py:184-187)."""
        self.scores.zero_()
        self.n_seen.zero_()

    def evict(self, budget, protected=0, n_action=None):
        """LRFU update, then keep + compact every request of the batch (a request within its
        budget keeps everything and is not moved).  n_action: action tokens scored this round
        per request (host ints; 0 = no action region, only decay).  protected is used at the
        batch's first eviction (a prefix count); afterwards the pins follow their tokens.
        Returns the compaction permutations (new -> old logical position), one per request."""
        from ..paged import _keep_mask_launch  # imported here: paged imports the kernels package
        cache, cfg = self.cache, self.cfg
        dev = self.ks.device
        R = len(self.reqs)
        L = cache.n_layers
        seqs = [cache.seq_used[r] for r in self.reqs]
        if max(seqs) > self.max_tokens:
            raise ValueError(f"a request holds {max(seqs)} tokens, more than max_tokens={self.max_tokens}")
        budgets = [max(b, 0) for b in _per_request(budget, R)]
        first = self.pin_counts is None
        counts = ([min(max(p, 0), s) for p, s in zip(_per_request(protected, R), seqs)] if first
                  else list(self.pin_counts))
        active = [True] * R if n_action is None else [int(n) > 0 for n in _per_request(n_action, R)]
        # within-budget requests keep every candidate (their compaction moves nothing)
        bud = [b if s - c > b else s for s, c, b in zip(seqs, counts, budgets)]
        kept = [min(c + b, s) for s, c, b in zip(seqs, counts, bud)]
        params = upload_i32(seqs + bud + counts + kept + [1 if a else 0 for a in active], dev)
        seq_dev, bud_dev, cnt_dev = params[:R], params[R:2 * R], params[2 * R:3 * R]
        kept_dev, act_dev = params[3 * R:4 * R], params[4 * R:]
        _lrfu_launch(self.scores, self.ks, seq_dev, cnt_dev if first else None, None if first else self.pins,
                     act_dev, max(seqs), cfg.decay, cfg.top_p, cfg.head_reduce)
        smax = max(seqs)
        ks4 = self.ks.unsqueeze(2)
        _, bits = _keep_mask_launch(ks4, L, 1, self.ks.stride(0), self.ks.stride(1), 0, R, seq_dev, bud_dev,
                                    cnt_dev if first else None, None if first else self.pins,
                                    0 if first else self.pins.stride(0), "mean", cache.block_size, smax, dev,
                                    want_keep=False)
        self._pins_alt.zero_()
        perm, _ = cache._compact_launch(self.reqs, bits, kept, None if first else self.pins,
                                        cnt_dev if first else None, pin_out=self._pins_alt)
        rc = _hip.lib().actkv_gather_tokens(
            self.ks.data_ptr(), self.ks.stride(0), self.ks.stride(1),
            self._ks_alt.data_ptr(), self._ks_alt.stride(0), self._ks_alt.stride(1),
            L, R, self.width, perm.data_ptr(), perm.stride(0), kept_dev.data_ptr(), _hip.stream(dev))
        _hip.check(rc, "actkv_gather_tokens")
        self.ks, self._ks_alt = self._ks_alt, self.ks
        self.pins, self._pins_alt = self._pins_alt, self.pins
        self.pin_counts = counts
        out = []
        for j, r in enumerate(self.reqs):
            pin = self.pins[j, : kept[j]]
            cache.pinned[r] = pin
            cache._pin_count[r] = (pin, pin._version, counts[j])
            out.append(perm[j, : kept[j]])
        return out
