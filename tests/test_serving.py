"""The HF paged backend's host logic on the CPU: a tiny Qwen3 served through PagedHFCache on a
CPU-resident PagedKVCache, with the oracle's paged attention standing in for the attention kernel
and a torch row write standing in for the append kernel, must
give the logits of the same model on eager attention with a contiguous DynamicCache (the
reference session's cache, actkv/hf/session.py:91-111): block allocation per step, per-layer
writes, RoPE positions, causal limits of a multi-token step, and the captured q and lse."""
import numpy as np
import pytest
import torch

transformers = pytest.importorskip("transformers")
from transformers import DynamicCache, Qwen3Config, Qwen3ForCausalLM  # noqa: E402

from actkv.hf import paged_session as ps  # noqa: E402
from actkv.paged import PagedKVCache  # noqa: E402
from oracle import reference as ref  # noqa: E402


def _tiny():
    cfg = Qwen3Config(vocab_size=101, hidden_size=64, intermediate_size=96, num_hidden_layers=3,
                      num_attention_heads=4, num_key_value_heads=2, head_dim=16, max_position_embeddings=512,
                      rope_theta=10000.0)
    torch.manual_seed(0)
    return Qwen3ForCausalLM(cfg).float().eval()


def _oracle_attention(q, kv_layer, bt, seq, scale, kv_len=None):
    table = bt.tolist()
    return ref.paged_attention(q.detach(), kv_layer, table, seq.tolist(), scale,
                               kv_len=None if kv_len is None else kv_len.tolist())


def _store_host(self, layer, st, key_states, value_states):
    """Test stand-in for the append launch on a CPU-resident cache: the step's rows written with
    torch at the slots the block table gives (reference paged.py:76-84, :93-97)."""
    b, hkv, n, d = key_states.shape
    bs = self.kv.block_size
    flat = self.kv.kv[layer].view(2, -1, hkv, d)
    for i, r in enumerate(self.reqs):
        pos = torch.arange(st.starts[i], st.starts[i] + n)
        slots = torch.tensor(self.kv.tables[r], dtype=torch.long)[pos // bs] * bs + pos % bs
        flat[0, slots] = key_states[i].transpose(0, 1).to(flat.dtype)
        flat[1, slots] = value_states[i].transpose(0, 1).to(flat.dtype)


def _rows_host(kv, req, layer):
    """K and V rows [S, Hkv, D] of a request in logical order, read through its block table."""
    s = kv.seq_used[req]
    return (ref.gather_k(kv.kv[layer], kv.tables[req], s), ref.gather_v(kv.kv[layer], kv.tables[req], s))


def _reference_logits(model, prompt, steps):
    """Eager attention and a DynamicCache, one sequence at a time."""
    model.set_attn_implementation("eager")
    out = []
    with torch.no_grad():
        cache = DynamicCache(config=model.config)
        lg = [model(input_ids=prompt[None], past_key_values=cache, use_cache=True).logits[0, -1]]
        for t in steps:
            lg.append(model(input_ids=t.view(1, 1), past_key_values=cache, use_cache=True).logits[0, -1])
        out.append(torch.stack(lg))
    return out[0], cache


def test_paged_backend_matches_eager_dynamic_cache(monkeypatch):
    model = _tiny()
    g = torch.Generator().manual_seed(1)
    B, n0, steps = 2, 11, 5
    prompts = torch.randint(0, 101, (B, n0), generator=g)
    toks = torch.randint(0, 101, (steps, B), generator=g)
    refs = [_reference_logits(model, prompts[b], toks[:, b]) for b in range(B)]

    monkeypatch.setattr(ps, "paged_decode_attention", _oracle_attention)
    monkeypatch.setattr(ps.PagedHFCache, "_store", _store_host)
    kv = PagedKVCache(24, 4, 2, 16, n_layers=3, dtype=torch.float32, device="cpu")
    kv.free = torch.randperm(24, generator=g).tolist()
    cache = ps.PagedHFCache(kv, [0, 1])
    model.set_attn_implementation(ps.register())
    seen = 0
    got = []
    with torch.no_grad():
        for ids in [prompts] + [toks[i][:, None] for i in range(steps)]:
            n = ids.shape[1]
            pos = torch.arange(seen, seen + n)[None].expand(B, n)
            cache.capture = n == 1
            out = model(input_ids=ids, past_key_values=cache, position_ids=pos,
                        attention_mask={"full_attention": None}, use_cache=True)
            got.append(out.logits[:, -1])
            seen += n
            if n == 1:      # the captured q and lse are the layer's query and its logsumexp
                st = cache.step
                assert sorted(st.q) == [0, 1, 2] and st.lse[2].shape == (B, 1, 4)
    got = torch.stack(got, 1)                      # [B, 1 + steps, V]
    for b in range(B):
        torch.testing.assert_close(got[b], refs[b][0], rtol=1e-4, atol=1e-4)
    # the paged rows are the DynamicCache's keys and values, every layer
    assert kv.seq_used == {0: n0 + steps, 1: n0 + steps}
    for b in range(B):
        dyn = refs[b][1]
        for layer in range(3):
            k, v = _rows_host(kv, b, layer)
            torch.testing.assert_close(k.transpose(0, 1), dyn.layers[layer].keys[0], rtol=0, atol=1e-6)
            torch.testing.assert_close(v.transpose(0, 1), dyn.layers[layer].values[0], rtol=0, atol=1e-6)
    # blocks came off the free stack request by request, step by step (as appends in order)
    assert len(kv.tables[0]) == len(kv.tables[1]) == -(-(n0 + steps) // 4)
    assert kv.used_blocks == 2 * 4


def test_multi_token_step_is_causal_and_positions_are_logical(monkeypatch):
    """Two tokens per step after a prompt: each query sees the prefix and the step's tokens up
    to itself, and RoPE takes logical positions that run past the physical length."""
    model = _tiny()
    g = torch.Generator().manual_seed(2)
    prompt = torch.randint(0, 101, (1, 6), generator=g)
    more = torch.randint(0, 101, (1, 3), generator=g)
    model.set_attn_implementation("eager")
    with torch.no_grad():
        dyn = DynamicCache(config=model.config)
        model(input_ids=prompt, past_key_values=dyn, position_ids=torch.arange(100, 106)[None], use_cache=True)
        want = model(input_ids=more, past_key_values=dyn, position_ids=torch.arange(106, 109)[None],
                     use_cache=True).logits[0]
    monkeypatch.setattr(ps, "paged_decode_attention", _oracle_attention)
    monkeypatch.setattr(ps.PagedHFCache, "_store", _store_host)
    kv = PagedKVCache(8, 4, 2, 16, n_layers=3, dtype=torch.float32, device="cpu")
    cache = ps.PagedHFCache(kv, [5])
    model.set_attn_implementation(ps.register())
    with torch.no_grad():
        model(input_ids=prompt, past_key_values=cache, position_ids=torch.arange(100, 106)[None],
              attention_mask={"full_attention": None}, use_cache=True)
        st_lim = None
        got = model(input_ids=more, past_key_values=cache, position_ids=torch.arange(106, 109)[None],
                    attention_mask={"full_attention": None}, use_cache=True).logits[0]
        st_lim = cache.step.kv_len.tolist()
    assert st_lim == [[7, 8, 9]]
    torch.testing.assert_close(got, want, rtol=1e-4, atol=1e-4)
    assert kv.seq_used[5] == 9 and cache.get_seq_length() == 9
    with pytest.raises(ValueError):
        model(input_ids=torch.zeros(2, 1, dtype=torch.long), past_key_values=cache,
              attention_mask={"full_attention": None}, use_cache=True)
