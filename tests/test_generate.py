"""The patched attention closure and generation loop
(samfurr/foveated_kv src/foveated_kv/mlx_generate.py:38-416) and the on-disk
archive format (disk_archive.py:127-222).

CPU: the closure's routing rules with stand-in layers (prefill pass-through,
layer counter and wrap, empty layers, dtype cast, spike stash, drain), the
formulation's immunity to the patch, the archive files.  GPU: a seeded tiny
LM decoding through the fused kernel, every layer call checked against the
reference formulation (dequant + concat + SDPA) of the same layer state, and
``generate_fused`` end to end with promotion."""

import types

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from foveated_kv_amd import generate as gen
from foveated_kv_amd.disk_archive import create_disk_archive, offload_cache_to_disk

ORIGINAL_SDPA = F.scaled_dot_product_attention


class StandInLayer:
    """Answers decode calls with a constant tensor tagged by layer."""

    def __init__(self, tag, Hkv=2, F_=5, D=8):
        self.tag = tag
        self.calls = 0
        self.near_k = torch.zeros(1, Hkv, 4, D, dtype=torch.float16)
        self.near_v = torch.ones(1, Hkv, 4, D, dtype=torch.float16)
        self.far_idx = torch.arange(F_, dtype=torch.int32).view(1, 1, -1).expand(1, Hkv, F_).contiguous()
        self.added = 0
        self.total_tokens = 40 + tag

    def add_token(self, k, v):
        self.added += k.shape[2]

    def attend_fused_with_spikes(self, q):
        self.calls += 1
        B, Hq = q.shape[0], q.shape[1]
        out = torch.full(q.shape, float(self.tag), dtype=torch.float16)
        return out, torch.full((B, Hq), self.tag % 2, dtype=torch.int32), torch.full((B, Hq), 100 + self.tag,
                                                                                    dtype=torch.int32)


class RecordingPipeline:
    def __init__(self):
        self.calls = []

    def drain_spikes(self, layer, flags, tokens, far_idx, step):
        self.calls.append((layer, flags.clone(), tokens.clone(), far_idx, step))


@pytest.fixture
def closure():
    gen.uninstall_fused_sdpa()
    yield gen
    gen.uninstall_fused_sdpa()
    assert F.scaled_dot_product_attention is ORIGINAL_SDPA


def _qkv(L, dtype=torch.float32, seed=0):
    g = torch.Generator().manual_seed(seed)
    q = torch.randn(1, 4, L, 8, generator=g).to(dtype)
    k = torch.randn(1, 4, L, 8, generator=g).to(dtype)
    v = torch.randn(1, 4, L, 8, generator=g).to(dtype)
    return q, k, v


def test_prefill_passes_through_and_decode_walks_layers(closure):
    layers = [StandInLayer(1), None, StandInLayer(3)]
    cache = types.SimpleNamespace(layers=layers)
    q, k, v = _qkv(5)
    want = ORIGINAL_SDPA(q, k, v, is_causal=True)
    closure.install_fused_sdpa(cache)
    assert F.scaled_dot_product_attention is not ORIGINAL_SDPA
    # q_len > 1: the original function, untouched, and no layer consumed
    got = F.scaled_dot_product_attention(q, k, v, is_causal=True)
    assert torch.equal(got, want)
    assert closure._fused_state._layer_counter == 0

    q1, k1, v1 = _qkv(1, seed=1)
    o0 = F.scaled_dot_product_attention(q1, k1, v1, scale=0.3)
    assert o0.dtype == torch.float32 and torch.all(o0 == 1.0)  # layer 0, cast to the query dtype
    o1 = F.scaled_dot_product_attention(q1, k1, v1)  # layer 1 is empty -> original
    assert torch.equal(o1, ORIGINAL_SDPA(q1, k1, v1))
    qb = q1.to(torch.bfloat16)
    o2 = F.scaled_dot_product_attention(qb, k1.to(torch.bfloat16), v1.to(torch.bfloat16))
    assert o2.dtype == torch.bfloat16 and torch.all(o2 == 3.0)
    o3 = F.scaled_dot_product_attention(q1, k1, v1)  # counter wraps modulo 3
    assert torch.all(o3 == 1.0)
    assert layers[0].calls == 2 and layers[2].calls == 1
    assert closure._fused_state._layer_counter == 4


def test_second_install_raises(closure):
    cache = types.SimpleNamespace(layers=[StandInLayer(0)])
    closure.install_fused_sdpa(cache)
    with pytest.raises(RuntimeError):
        closure.install_fused_sdpa(cache)
    closure.uninstall_fused_sdpa()
    closure.uninstall_fused_sdpa()  # idempotent
    assert F.scaled_dot_product_attention is ORIGINAL_SDPA


def test_drain_hands_stashed_spikes_to_the_pipeline(closure):
    layers = [StandInLayer(1), None, StandInLayer(2)]
    cache = types.SimpleNamespace(layers=layers)
    wrappers = closure.install_fused_attention(None, cache)
    assert wrappers[1] is None and wrappers[0].layer_idx == 0 and wrappers[2].layer_idx == 2
    q1, k1, v1 = _qkv(1)
    for _ in range(3):
        F.scaled_dot_product_attention(q1, k1, v1)
    assert wrappers[0]._spike_flags is not None and wrappers[2]._spike_tokens is not None
    pipe = RecordingPipeline()
    closure.drain_spikes(wrappers, pipe, 7)
    assert closure._fused_state._layer_counter == 0
    assert closure._fused_state._decode_step == 1
    assert [c[0] for c in pipe.calls] == [0, 2]
    for (layer, flags, tokens, far_idx, step), lay in zip(pipe.calls, (layers[0], layers[2])):
        assert step == 7 and far_idx is lay.far_idx
        assert torch.all(flags == lay.tag % 2) and torch.all(tokens == 100 + lay.tag)
    assert all(w is None or (w._spike_flags is None and w._spike_tokens is None) for w in wrappers)
    # no pipeline: only the counter moves and the stash is kept
    # (mlx_generate.py:219-220 returns before touching the wrappers) ...
    F.scaled_dot_product_attention(q1, k1, v1)
    closure.drain_spikes(wrappers, None, 8)
    assert closure._fused_state._layer_counter == 0 and closure._fused_state._decode_step == 2
    assert wrappers[0]._spike_flags is not None
    # ... so the next drain with a pipeline hands it over
    closure.drain_spikes(wrappers, pipe, 9)
    assert [(c[0], c[4]) for c in pipe.calls[2:]] == [(0, 9)]
    closure.drain_spikes(wrappers, pipe, 10)
    assert len(pipe.calls) == 3


def test_fused_cache_wrapper_interface():
    lay = StandInLayer(5)
    w = gen.FusedCacheWrapper(lay, 3)
    assert w.offset == lay.total_tokens
    k = torch.randn(1, 2, 1, 8)
    v = torch.randn(1, 2, 1, 8)
    rk, rv = w.update_and_fetch(k, v)
    assert rk is k and rv is v and lay.added == 1 and w.offset == lay.total_tokens + 1
    nk, nv = w.state
    assert nk is lay.near_k and nv is lay.near_v
    fi = w.far_idx_host()
    assert fi.dtype == np.int32 and fi.shape == (1, 2, 5) and w.far_idx_host() is fi


def test_formulation_is_immune_to_the_patch(closure):
    from foveated_kv_amd.tier_cache import standard_attention

    q1, k1, v1 = _qkv(1, seed=3)
    want = standard_attention(q1, k1, v1)
    closure.install_fused_sdpa(types.SimpleNamespace(layers=[StandInLayer(1)]))
    got = standard_attention(q1, k1, v1)
    assert torch.equal(got, want)
    assert closure._fused_state._layer_counter == 0


def test_kv_cache_appends():
    c = gen.KVCache()
    a = torch.randn(1, 2, 3, 4)
    b = torch.randn(1, 2, 1, 4)
    k, v = c.update_and_fetch(a, a + 1)
    assert c.offset == 3 and torch.equal(k, a)
    k, v = c.update_and_fetch(b, b + 1)
    assert c.offset == 4 and torch.equal(k, torch.cat([a, b], 2)) and torch.equal(v, torch.cat([a, b], 2) + 1)
    model = types.SimpleNamespace(layers=[0, 0, 0])
    assert len(gen.make_prompt_cache(model)) == 3


def test_disk_archive_files_round_trip(tmp_path):
    g = torch.Generator().manual_seed(5)
    H, S, D = 3, 17, 16
    ak = torch.randn(1, H, S, D, generator=g).half()
    av = torch.randn(1, H, S, D, generator=g).half()
    idx = torch.arange(4, 4 + S, dtype=torch.int32).view(1, 1, S).expand(1, H, S).contiguous()
    a = create_disk_archive(ak, av, idx, 2, tmp_path)
    assert a.path_k.endswith("archive_k_layer2.bin") and a.path_v.endswith("archive_v_layer2.bin")
    raw = np.fromfile(a.path_k, dtype="<f2").reshape(H, S, D)
    assert np.array_equal(raw.view(np.uint16), ak[0].numpy().view(np.uint16))
    k, v = a.promote(1, 9)
    assert torch.equal(k.reshape(-1), ak[0, 1, 9]) and torch.equal(v.reshape(-1), av[0, 1, 9])
    kb, vb = a.promote_batch(2, [0, 16, 3])
    assert kb.shape == (1, 1, 3, D) and torch.equal(kb[0, 0], ak[0, 2, [0, 16, 3]])
    assert a.promote_batch(0, [])[0].shape == (1, 1, 0, D)
    s = a.score_boundary_tokens(0, np.ones(D, np.float32), [1, 2])
    assert np.allclose(s, ak[0, 0, [1, 2]].float().sum(-1).numpy(), atol=1e-3)
    assert a.disk_bytes() == H * S * D * 4
    assert create_disk_archive(ak[:, :, :0], av[:, :, :0], idx[:, :, :0], 3, tmp_path) is None
    with pytest.raises(ValueError):
        create_disk_archive(ak.expand(2, -1, -1, -1), av.expand(2, -1, -1, -1), idx, 4, tmp_path)


def test_offload_cache_to_disk_leaves_placeholders(tmp_path):
    g = torch.Generator().manual_seed(6)
    lay = types.SimpleNamespace(archive_k=torch.randn(1, 2, 5, 8, generator=g).half(),
                                archive_v=torch.randn(1, 2, 5, 8, generator=g).half(),
                                archive_idx=torch.zeros(1, 2, 5, dtype=torch.int32))
    keep = lay.archive_k.clone()
    arcs = offload_cache_to_disk(types.SimpleNamespace(layers=[None, lay]), tmp_path)
    assert arcs[0] is None and arcs[1].S_arc == 5
    assert lay.archive_k.shape == (1, 2, 0, 8) and lay.archive_v.shape == (1, 2, 0, 8)
    assert torch.equal(arcs[1].promote(1, 4)[0].reshape(-1), keep[0, 1, 4])


# ---------------------------------------------------------------------------
# GPU: the closure on a real model
# ---------------------------------------------------------------------------


def _prompt(n, seed):
    rng = np.random.default_rng(seed)
    return "".join(chr(c) for c in rng.integers(97, 123, size=n))


def _stats(a, b):
    a = a.double().reshape(-1)
    b = b.double().reshape(-1)
    return float((a - b).abs().max()), float(torch.nn.functional.cosine_similarity(a, b, dim=0))


@pytest.mark.gpu
def test_decode_closure_matches_formulation_every_layer(closure):
    from _tiny_lm import ByteTokenizer, TinyLM

    dev = torch.device("cuda:0")
    model = TinyLM(seed=11).to(dev).eval()
    tok = ByteTokenizer()
    print("case: tiny LM S=600 Hq=8 Hkv=2 D=64, 6 decode steps", flush=True)
    ids = torch.tensor(tok.encode(_prompt(600, 1)), device=dev).reshape(1, -1)
    fov_cache, logits, _ = gen.prefill_and_compress(model, ids)
    wrappers = closure.install_fused_attention(model, fov_cache)
    checks = []
    for lay in fov_cache.layers:
        fused = lay.attend_fused_with_spikes

        def checked(q, lay=lay, fused=fused):
            want = lay.attend(q)  # same layer state: the new token is already in the decode buffer
            out, flags, tokens = fused(q)
            checks.append((want, out.to(q.dtype), flags, tokens))
            return out, flags, tokens

        lay.attend_fused_with_spikes = checked
    nxt = logits[:, -1, :]
    with torch.no_grad():
        for step in range(6):
            t = torch.argmax(nxt, dim=-1)
            closure.drain_spikes(wrappers, None, step)
            nxt = model(t.reshape(1, 1), cache=wrappers)[:, -1, :]
    torch.cuda.synchronize()
    assert len(checks) == 6 * len(fov_cache.layers)
    for want, got, flags, tokens in checks:
        assert got.dtype == torch.float32 and got.shape == want.shape == (1, 8, 1, 64)
        mx, cs = _stats(got, want)
        assert mx <= 2e-3 and cs >= 0.9999, (mx, cs)
        assert flags.shape == (1, 8) and tokens.shape == (1, 8)
    assert all(w.fov_layer.decode_k.shape[2] == 6 for w in wrappers)
    assert wrappers[0].offset == 600 + 6


@pytest.mark.gpu
def test_generate_fused_tokens_match_formulation_decode(closure):
    from _tiny_lm import ByteTokenizer, TinyLM

    dev = torch.device("cuda:0")
    model = TinyLM(seed=12).to(dev).eval()
    tok = ByteTokenizer()
    prompt = _prompt(500, 2)
    print("case: generate_fused without promotion vs formulation greedy, 8 tokens", flush=True)
    text, stats = gen.generate_fused(model, tok, prompt, max_tokens=8, enable_promotion=False)
    assert stats["generated_tokens"] == 8 and stats["mem_archive_after_mb"] == 0.0
    assert closure._fused_state._installed is False

    ids = torch.tensor(tok.encode(prompt), device=dev).reshape(1, -1)
    fov_cache, logits, _ = gen.prefill_and_compress(model, ids)
    for lay in fov_cache.layers:
        lay.attend_fused_with_spikes = lambda q, lay=lay: (lay.attend(q), None, None)
    wrappers = closure.install_fused_attention(model, fov_cache)
    want = []
    nxt = logits[:, -1, :]
    with torch.no_grad():
        for step in range(8):
            t = torch.argmax(nxt, dim=-1)
            want.append(int(t))
            closure.drain_spikes(wrappers, None, step)
            nxt = model(t.reshape(1, 1), cache=wrappers)[:, -1, :]
    assert text == tok.decode(want)


@pytest.mark.gpu
def test_generate_fused_promotes_spiking_far_tokens(closure, tmp_path):
    from _tiny_lm import ByteTokenizer, TinyLM

    dev = torch.device("cuda:0")
    # large q/k gain -> scores spread far beyond the 10.0 spike margin
    model = TinyLM(seed=13, qk_gain=3.0).to(dev).eval()
    tok = ByteTokenizer()
    print("case: generate_fused with promotion, qk_gain 3, 12 tokens", flush=True)
    text, stats = gen.generate_fused(model, tok, _prompt(700, 3), max_tokens=12,
                                     disk_archive_dir=str(tmp_path / "arc"), enable_promotion=True)
    assert stats["generated_tokens"] == 12
    assert stats["spikes_detected"] > 0
    assert stats["promotions_completed"] > 0
    assert stats["promotions_completed"] + stats["promotions_headroom_full"] <= stats["spikes_queued"]
    assert not (tmp_path / "arc").exists()
    # the drain on the device promotes the same tokens and generates the same text
    text_d, stats_d = gen.generate_fused(model, tok, _prompt(700, 3), max_tokens=12,
                                         disk_archive_dir=str(tmp_path / "arc2"), enable_promotion=True,
                                         device_drain=True)
    assert text_d == text
    for key in ("spikes_detected", "spikes_queued", "spikes_deduplicated", "spikes_cooled_down",
                "promotions_completed", "promotions_headroom_full"):
        assert stats_d[key] == stats[key], key


class _EosTokenizer:
    """ByteTokenizer with an end-of-sequence id."""

    def __init__(self, base, eos):
        self.base = base
        self.eos_token_id = eos

    def encode(self, text):
        return self.base.encode(text)

    def decode(self, ids):
        return self.base.decode(ids)


@pytest.mark.gpu
def test_generate_graph_matches_eager_tokens_and_promotions(closure, tmp_path):
    """One HIP graph per model decode step (device step state, device decode
    count, device drain) generates the eager closure's tokens and promotes
    the same rows; with an EOS id both stop at the same token."""
    from _tiny_lm import ByteTokenizer, TinyLM

    dev = torch.device("cuda:0")
    model = TinyLM(seed=14, qk_gain=3.0).to(dev).eval()
    tok = ByteTokenizer()
    prompt = _prompt(700, 4)
    print("case: generate_fused graph vs eager device drain, qk_gain 3, 24 tokens", flush=True)
    text_e, st_e = gen.generate_fused(model, tok, prompt, max_tokens=24, disk_archive_dir=str(tmp_path / "a"),
                                      device_drain=True)
    text_g, st_g = gen.generate_fused(model, tok, prompt, max_tokens=24, disk_archive_dir=str(tmp_path / "b"),
                                      graph=True)
    assert st_g["graph"] and st_g["model_calls"] == st_e["model_calls"] == 24
    assert text_g == text_e
    assert st_e["promotions_completed"] > 0
    for key in ("spikes_detected", "spikes_queued", "spikes_deduplicated", "spikes_cooled_down",
                "promotions_completed", "promotions_headroom_full"):
        assert st_g[key] == st_e[key], key
    assert closure._fused_state._installed is False and closure._fused_state._dev is None
    # an EOS id taken from the middle of the generated text: both loops stop there
    ids = [int(x) for x in text_e.split()]
    eos = ids[17]
    want = ids[:ids.index(eos)]
    print(f"case: graph vs eager with EOS id {eos} (first at {len(want)})", flush=True)
    etok = _EosTokenizer(tok, eos)
    text_e2, st_e2 = gen.generate_fused(model, etok, prompt, max_tokens=24, enable_promotion=True,
                                        device_drain=True)
    text_g2, st_g2 = gen.generate_fused(model, etok, prompt, max_tokens=24, enable_promotion=True, graph=True)
    assert text_e2 == text_g2 == tok.decode(want)
    assert st_g2["generated_tokens"] == len(want)


@pytest.mark.gpu
def test_graph_decode_leaves_host_state_consistent(closure):
    """After a graph decode the caches hold the steps on the host again: the
    decode buffers' row counts and the wrappers' offsets advance by the
    model calls made, and the buffered rows are the ones eager decode
    appends."""
    from _tiny_lm import ByteTokenizer, TinyLM

    dev = torch.device("cuda:0")
    model = TinyLM(seed=15).to(dev).eval()
    tok = ByteTokenizer()
    ids = torch.tensor(tok.encode(_prompt(400, 5)), device=dev).reshape(1, -1)
    print("case: graph decode host state, 6 steps", flush=True)
    caches = []
    for graph in (False, True):
        fov_cache, logits, _ = gen.prefill_and_compress(model, ids)
        wrappers = closure.install_fused_attention(model, fov_cache)
        nxt = logits[:, -1, :]
        with torch.no_grad():
            if graph:
                toks, calls, _ = gen._decode_graph(model, wrappers, None, nxt, 6, None, dev)
                assert calls == 6
            else:
                toks = []
                for step in range(6):
                    t = torch.argmax(nxt, dim=-1)
                    toks.append(int(t))
                    closure.drain_spikes(wrappers, None, step)
                    nxt = model(t.reshape(1, 1), cache=wrappers)[:, -1, :]
        torch.cuda.synchronize()
        closure.uninstall_fused_attention(model)
        caches.append((toks, [(w.offset, w.fov_layer.decode_k.clone(), w.fov_layer.decode_v.clone())
                              for w in wrappers]))
    (te, ce), (tg, cg) = caches
    assert te == tg
    for (oe, ke, ve), (og, kg, vg) in zip(ce, cg):
        assert oe == og == 400 + 6
        assert ke.shape == kg.shape and ke.shape[2] == 6
        assert torch.equal(ke, kg) and torch.equal(ve, vg)
