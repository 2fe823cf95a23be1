"""GPU tests of the Python surface over the HIP kernels (torch binding `barqtrain_cuda`).

* The reference's cache-layer API (kv_cache.py:37-194) on GPU tensors, driven by seeded random
  programs, against the CPU oracle -- bit-exact on raw element bits.
* HIP-graph capture of a decode step (every layer's fused append + gather recorded once,
  lengths read on the device): every replay, with eager work and synchronisations between
  replays, against the oracle.
* Hugging Face `generate` with the paged cache on the GPU: same tokens and bit-identical logits
  as transformers' DynamicCache.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from kvgen import hf_layout, to_bits
from mirror import DeviceMirror
from oracle.kv_oracle import DenseLayerOracle

pytestmark = pytest.mark.gpu


def assert_bits(got: torch.Tensor, want: np.ndarray, what: str):
    g = to_bits(got)
    assert g.shape == want.shape, (what, g.shape, want.shape)
    if not np.array_equal(g, want):
        bad = np.argwhere(g != want)
        raise AssertionError(f"{what}: {len(bad)} elements differ, first at {bad[0].tolist()}")


@pytest.mark.parametrize("seed", [0, 1, 2])
def test_layer_api_random_program(hip, seed):
    """update (ragged batches, multi-token), current_tensors, crop (also negative), beam select /
    repeat, reset and row release through BarqPagedKVCacheLayer on cuda:0."""
    from barqtrain_amd.kv_cache import BarqPagedKVCacheLayer

    H, D, P, dtype = 8, 128, 16, torch.bfloat16
    Bmax, cap = 4, 72
    rng = np.random.default_rng(100 + seed)
    gen = torch.Generator().manual_seed(seed)
    layer = BarqPagedKVCacheLayer(max_batch_size=Bmax, max_cache_len=cap, page_size=P)
    oracle = DenseLayerOracle(Bmax, cap, P)
    for it in range(40):
        r = rng.random()
        if r < 0.55 or not oracle.is_initialized:
            b = int(rng.integers(1, layer.max_batch_size + 1))
            t = int(rng.integers(1, 20)) if rng.random() < 0.3 else 1
            if oracle.is_initialized and int(oracle.seq_lens[:b].max()) + t > cap:
                continue
            k = hf_layout(b, H, t, D, dtype, gen)
            v = hf_layout(b, H, t, D, dtype, gen)
            gk, gv = layer.update(k.cuda(), v.cuda())
            ok, ov = oracle.update(to_bits(k), to_bits(v))
            assert_bits(gk, ok, f"it{it} update K")
            assert_bits(gv, ov, f"it{it} update V")
        elif r < 0.65:
            m = int(rng.integers(-8, cap))
            layer.crop(m)
            oracle.crop(m)
        elif r < 0.72 and layer.current_batch_size:
            rows = rng.integers(0, layer.current_batch_size, size=layer.current_batch_size).tolist()
            layer.batch_select_indices(torch.tensor(rows))
            oracle.batch_select_indices(rows)
        elif r < 0.76 and layer.current_batch_size and layer.current_batch_size * 2 <= 8:
            layer.batch_repeat_interleave(2)
            oracle.batch_repeat_interleave(2)
        elif r < 0.82:
            rows = sorted(rng.choice(layer.max_batch_size, size=1, replace=False).tolist())
            layer.free_rows(rows)
            oracle.release_rows(rows)
        elif r < 0.85:
            layer.reset()
            oracle.reset()
        if layer.current_batch_size:
            assert layer.get_seq_length() == oracle.get_seq_length()
            ok, ov = oracle.current_tensors()
            gk, gv = layer.current_tensors()
            assert_bits(gk, ok, f"it{it} current K")
            assert_bits(gv, ov, f"it{it} current V")
    assert layer.pool.errors() == 0


def test_graph_replays_match_oracle(hip):
    """One captured decode step (3 layers, batch 4), replayed 24 times; between replays the
    program does its own eager work (random tensors, reductions, an eager gather) and
    synchronises; every replay's K/V views are compared with the oracle."""
    from barqtrain_amd.graph import CapturedDecodeStep
    from barqtrain_amd.paged import PagePool

    L, B, H, D, P, prefill, steps = 3, 4, 8, 128, 16, 40, 24
    cap = prefill + steps
    dev = torch.device("cuda", 0)
    gen = torch.Generator().manual_seed(7)
    pools = [PagePool(max_batch=B, max_blocks=-(-cap // P), page_size=P, kv_heads=H, head_dim=D,
                      dtype=torch.bfloat16, device=dev) for _ in range(L)]
    oracles = [DenseLayerOracle(B, cap, P) for _ in range(L)]
    for pool, oracle in zip(pools, oracles):
        k = hf_layout(B, H, prefill, D, torch.bfloat16, gen)
        v = hf_layout(B, H, prefill, D, torch.bfloat16, gen)
        pool.update(k.to(dev), v.to(dev))
        oracle.update(to_bits(k), to_bits(v))
    kin = torch.zeros((L, B, H, 1, D), dtype=torch.bfloat16, device=dev)
    vin = torch.zeros_like(kin)
    step = CapturedDecodeStep(pools, B, 1, inputs=(kin, vin))
    torch.cuda.synchronize()
    noise = torch.Generator(device=dev).manual_seed(3)
    for s in range(steps):
        ks = [hf_layout(B, H, 1, D, torch.bfloat16, gen) for _ in range(L)]
        vs = [hf_layout(B, H, 1, D, torch.bfloat16, gen) for _ in range(L)]
        for layer in range(L):
            kin[layer].copy_(ks[layer].to(dev))
            vin[layer].copy_(vs[layer].to(dev))
        scratch = torch.randn((1 << 20,), generator=noise, device=dev)  # eager work between replays
        _ = scratch.sum().item()
        outs = step.replay()
        torch.cuda.synchronize()
        for layer in range(L):
            ok, ov = oracles[layer].update(to_bits(ks[layer]), to_bits(vs[layer]))
            assert_bits(outs[layer][0], ok, f"replay {s} layer {layer} K")
            assert_bits(outs[layer][1], ov, f"replay {s} layer {layer} V")
        if s % 8 == 7:  # an eager gather between replays reads the same state
            gk, gv = pools[0].gather(B)
            ok, ov = oracles[0].current_tensors()
            assert_bits(gk, ok, f"eager gather after replay {s}")
    assert all(p.errors() == 0 for p in pools)
    assert [int(x) for x in pools[0].seq_lens.cpu()] == [cap] * B


def test_config2_all_layers_captured_every_step(hip):
    """The benchmark's C2 step as it runs there: 32 layers of 16 rows x 8 KV heads x 128, bf16,
    page 16, prefill 512, then 256 replays of one captured decode step.  Every replay's K/V of
    every layer against the device mirror; every layer against the oracle after the last replay
    (and the mirror with it)."""
    from barqtrain_amd.graph import CapturedDecodeStep
    from barqtrain_amd.paged import PagePool

    L, B, H, D, P, prefill, steps = 32, 16, 8, 128, 16, 512, 256
    cap = prefill + steps
    dev = torch.device("cuda", 0)
    bf16 = torch.bfloat16
    gen = torch.Generator(device=dev).manual_seed(2002)

    def tokens(T):  # [B, H, T, D] view of [B, T, H, D], as HF hands K/V to the cache
        return torch.randn((B, T, H, D), generator=gen, device=dev).to(bf16).transpose(1, 2)

    pools = [PagePool(max_batch=B, max_blocks=cap // P, page_size=P, kv_heads=H, head_dim=D, dtype=bf16,
                      device=dev) for _ in range(L)]
    mirrors = [DeviceMirror(B, H, cap, D, bf16) for _ in range(L)]
    oracles = [DenseLayerOracle(B, cap, P) for _ in range(L)]
    for pool, mirror, oracle in zip(pools, mirrors, oracles):
        k, v = tokens(prefill), tokens(prefill)
        mirror.append(k, v)
        mirror.check(pool.update(k, v), "prefill")
        oracle.append(to_bits(k), to_bits(v))
    kin = torch.zeros((L, B, H, 1, D), dtype=bf16, device=dev)
    vin = torch.zeros_like(kin)
    step = CapturedDecodeStep(pools, B, 1, inputs=(kin, vin))
    step.prepare(range(prefill + 1, cap + 1))
    outs = None
    for s in range(steps):
        kin.copy_(torch.randn(kin.shape, generator=gen, device=dev).to(bf16))
        vin.copy_(torch.randn(vin.shape, generator=gen, device=dev).to(bf16))
        outs = step.replay()
        kh, vh = to_bits(kin), to_bits(vin)
        for layer in range(L):
            mirrors[layer].append(kin[layer], vin[layer])
            mirrors[layer].check(outs[layer], f"replay {s} layer {layer}")
            oracles[layer].append(kh[layer], vh[layer])
    for layer in range(L):
        ok, ov = oracles[layer].current_tensors()
        assert_bits(outs[layer][0], ok, f"layer {layer} K after {steps} replays")
        assert_bits(outs[layer][1], ov, f"layer {layer} V after {steps} replays")
    assert all(p.errors() == 0 for p in pools)


def tiny_llama(seed=0):
    from transformers import LlamaConfig, LlamaForCausalLM

    torch.manual_seed(seed)
    # head_dim 128, 2 KV heads, fp32: a 1 KiB K row per token, the kernels' wave-uniform path
    cfg = LlamaConfig(vocab_size=512, hidden_size=512, intermediate_size=512, num_hidden_layers=2,
                      num_attention_heads=4, num_key_value_heads=2, max_position_embeddings=1024,
                      pad_token_id=0, eos_token_id=None, attn_implementation="eager")
    return LlamaForCausalLM(cfg).eval(), cfg


def test_generate_on_gpu_matches_dynamic_cache(hip, monkeypatch):
    pytest.importorskip("transformers")
    from transformers.cache_utils import DynamicCache

    from barqtrain import create_paged_kv_cache, patch_inference

    model, cfg = tiny_llama()
    model = model.to("cuda")
    ids = torch.randint(1, 512, (3, 21), generator=torch.Generator().manual_seed(2)).to("cuda")
    new = 40

    def decode(cache):
        out = model.generate(ids, attention_mask=torch.ones_like(ids), max_new_tokens=new, do_sample=False,
                             past_key_values=cache, return_dict_in_generate=True, output_logits=True)
        return out.sequences, torch.stack(out.logits)

    ref_seq, ref_logits = decode(DynamicCache(config=cfg))
    cache = create_paged_kv_cache(model, max_batch_size=3, max_cache_len=21 + new, page_size=16)
    seq, logits = decode(cache)
    assert torch.equal(seq, ref_seq)
    assert torch.equal(logits.view(torch.int32), ref_logits.view(torch.int32))
    assert all(layer.pool.on_gpu and layer.pool.errors() == 0 for layer in cache.layers)

    # the reference's injection route: patch_inference wraps generate and supplies the cache
    monkeypatch.setenv("BARQTRAIN_PAGED_KV_MIN_CACHE_LEN", "0")
    patch_inference(model)
    model.config._attn_implementation = "eager"
    out = model.generate(ids, attention_mask=torch.ones_like(ids), max_new_tokens=new, do_sample=False)
    assert model._barqtrain_last_generate_used_paged_kv is True
    assert torch.equal(out, ref_seq)


def bf16_llama(seed=0):
    from transformers import LlamaConfig, LlamaForCausalLM

    torch.manual_seed(seed)
    # 8 query heads over 2 kv heads (G = 4, the Llama-3 ratio), head_dim 128, bf16
    cfg = LlamaConfig(vocab_size=512, hidden_size=1024, intermediate_size=1024, num_hidden_layers=2,
                      num_attention_heads=8, num_key_value_heads=2, max_position_embeddings=1024,
                      pad_token_id=0, eos_token_id=None)
    return LlamaForCausalLM(cfg).to(torch.bfloat16).eval(), cfg


def qwen2_small_head(seed=0):
    from transformers import Qwen2Config, Qwen2ForCausalLM

    torch.manual_seed(seed)
    # Qwen2-0.5B's attention geometry (the reference's benchmark model): 14 query heads over 2 kv
    # heads (G = 7), head_dim 64, q/k/v biases; fewer layers and a small vocabulary
    cfg = Qwen2Config(vocab_size=512, hidden_size=896, intermediate_size=1024, num_hidden_layers=2,
                      num_attention_heads=14, num_key_value_heads=2, max_position_embeddings=1024,
                      pad_token_id=0, eos_token_id=None)
    return Qwen2ForCausalLM(cfg).to(torch.bfloat16).eval(), cfg


def wide_head(seed=0):
    from transformers import LlamaConfig, LlamaForCausalLM

    torch.manual_seed(seed)
    # Gemma-2B's attention geometry: 8 query heads over 1 kv head (G = 8), head_dim 256
    cfg = LlamaConfig(vocab_size=512, hidden_size=1024, intermediate_size=1024, num_hidden_layers=2,
                      num_attention_heads=8, num_key_value_heads=1, head_dim=256, max_position_embeddings=1024,
                      pad_token_id=0, eos_token_id=None)
    return LlamaForCausalLM(cfg).to(torch.bfloat16).eval(), cfg


@pytest.mark.parametrize("factory", [bf16_llama, qwen2_small_head, wide_head],
                         ids=["llama_d128_g4", "qwen2_d64_g7", "llama_d256_g8"])
def test_paged_attention_decode_in_a_model(hip, monkeypatch, factory):
    """A bf16 model whose decode steps read K/V from the pages (the kernel) against the same
    model on the gather + fp32 attention path, token by token on one sequence: logits agree to
    bf16 rounding.  Then generate() through patch_inference(paged_attention=True).  Head sizes 128
    (Llama-3 ratio), 64 (Qwen2-0.5B geometry) and 256 (Gemma-2B geometry)."""
    pytest.importorskip("transformers")
    from barqtrain import create_paged_kv_cache, patch_inference
    from barqtrain_amd import attention

    model, cfg = factory()
    model = model.to("cuda")
    attention.enable_paged_attention(model)
    gen = torch.Generator().manual_seed(5)
    prompt, new = 37, 24
    seq = torch.randint(1, 512, (3, prompt + new), generator=gen).to("cuda")

    from barqtrain_amd.paged import PagePool

    calls = []
    attend = PagePool.attend
    monkeypatch.setattr(PagePool, "attend", lambda self, *a, **k: calls.append(1) or attend(self, *a, **k))

    def run(kernel: bool):
        monkeypatch.setattr(attention, "_KERNEL_MAX_ROWS", 16 if kernel else 0)
        # the reference attention is the fp32 one, not the fused bf16 SDPA the route takes
        monkeypatch.setattr(attention, "_sdpa_attention", lambda *a: None)
        cache = create_paged_kv_cache(model, max_batch_size=3, max_cache_len=prompt + new, page_size=16)
        steps = []
        with torch.no_grad():
            out = model(seq[:, :prompt], past_key_values=cache, use_cache=True)
            steps.append(out.logits[:, -1].float())
            for t in range(new - 1):
                out = model(seq[:, prompt + t:prompt + t + 1], past_key_values=cache, use_cache=True)
                steps.append(out.logits[:, -1].float())
        assert all(layer.pool.errors() == 0 for layer in cache.layers)
        return torch.stack(steps)

    fused = run(True)
    assert len(calls) == cfg.num_hidden_layers * (new - 1), "decode steps ran the kernel"
    reference = run(False)
    assert len(calls) == cfg.num_hidden_layers * (new - 1), "the fallback ran no kernel"
    scale = reference.abs().max().item()
    err = (fused - reference).abs().max().item()
    assert err <= 0.02 * scale, f"logits differ by {err} (scale {scale})"
    assert (fused.argmax(-1) == reference.argmax(-1)).float().mean().item() >= 0.9

    monkeypatch.undo()
    monkeypatch.setenv("BARQTRAIN_PAGED_KV_MIN_CACHE_LEN", "0")
    patch_inference(model, paged_attention=True)
    out = model.generate(seq[:, :prompt], attention_mask=torch.ones_like(seq[:, :prompt]), max_new_tokens=8,
                         do_sample=False)
    assert model._barqtrain_last_generate_used_paged_kv is True
    assert out.shape == (3, prompt + 8)


def test_graph_recaptured_after_pool_tensors_move(hip):
    """A captured step whose pool is moved off the GPU and back (PagePool.to: new device
    tensors) captures its graphs again instead of replaying launches on the freed memory."""
    from barqtrain_amd.graph import CapturedDecodeStep
    from barqtrain_amd.paged import PagePool

    L, B, H, D, P, prefill, steps = 2, 3, 8, 128, 16, 20, 8
    cap = prefill + steps
    dev = torch.device("cuda", 0)
    gen = torch.Generator().manual_seed(9)
    pools = [PagePool(max_batch=B, max_blocks=-(-cap // P), page_size=P, kv_heads=H, head_dim=D,
                      dtype=torch.bfloat16, device=dev) for _ in range(L)]
    oracles = [DenseLayerOracle(B, cap, P) for _ in range(L)]
    for pool, oracle in zip(pools, oracles):
        k = hf_layout(B, H, prefill, D, torch.bfloat16, gen)
        pool.update(k.to(dev), k.to(dev))
        oracle.update(to_bits(k), to_bits(k))
    kin = torch.zeros((L, B, H, 1, D), dtype=torch.bfloat16, device=dev)
    step = CapturedDecodeStep(pools, B, 1, inputs=(kin, kin))
    for s in range(steps):
        if s == steps // 2:
            torch.cuda.synchronize()
            pools[1].to("cpu")
            torch.cuda.synchronize()
            pools[1].to(dev)
            torch.cuda.synchronize()
        ks = [hf_layout(B, H, 1, D, torch.bfloat16, gen) for _ in range(L)]
        for layer in range(L):
            kin[layer].copy_(ks[layer].to(dev))
        outs = step.replay()
        torch.cuda.synchronize()
        for layer in range(L):
            ok, ov = oracles[layer].update(to_bits(ks[layer]), to_bits(ks[layer]))
            assert_bits(outs[layer][0], ok, f"replay {s} layer {layer} K")
            assert_bits(pools[layer].gather(B)[1], ov, f"replay {s} layer {layer} V (eager gather)")
    assert all(p.errors() == 0 for p in pools)


def small_head_llama(seed=0):
    from transformers import LlamaConfig, LlamaForCausalLM

    torch.manual_seed(seed)
    # head_dim 64 with 4 query heads over 2 kv heads
    cfg = LlamaConfig(vocab_size=512, hidden_size=256, intermediate_size=512, num_hidden_layers=2,
                      num_attention_heads=4, num_key_value_heads=2, max_position_embeddings=1024,
                      pad_token_id=0, eos_token_id=None)
    return LlamaForCausalLM(cfg).to(torch.bfloat16).eval(), cfg


def test_paged_route_head_dim_64_and_padded_batch(hip, monkeypatch):
    """The "barq_paged" route for calls the decode kernel does not take -- a left-padded batch (a
    mask), here with head_dim 64 -- runs torch's fused SDPA over the gathered K/V.  Against the same
    route with the fp32 attention (a reference free of bf16 batched products): prefill logits
    agree to bf16 rounding and greedy tokens agree."""
    pytest.importorskip("transformers")
    from barqtrain import create_paged_kv_cache
    from barqtrain_amd import attention

    model, cfg = small_head_llama()
    model = model.to("cuda")
    attention.enable_paged_attention(model)
    ids = torch.randint(1, 512, (3, 29), generator=torch.Generator().manual_seed(6)).to("cuda")
    mask = torch.ones_like(ids)
    mask[1, :5] = 0  # row 1 left-padded
    mask[2, :11] = 0
    new = 16
    sdpa = attention._sdpa_attention
    fused = []

    def decode(use_sdpa: bool):
        monkeypatch.setattr(attention, "_sdpa_attention",
                            (lambda *a: fused.append(1) or sdpa(*a)) if use_sdpa else (lambda *a: None))
        cache = create_paged_kv_cache(model, max_batch_size=3, max_cache_len=29 + new, page_size=16)
        out = model.generate(ids, attention_mask=mask, max_new_tokens=new, do_sample=False, past_key_values=cache,
                             return_dict_in_generate=True, output_logits=True)
        assert all(layer.pool.errors() == 0 for layer in cache.layers)
        return out.sequences, torch.stack(out.logits).float()

    seq, logits = decode(True)
    assert len(fused) >= cfg.num_hidden_layers * new, "every attention call ran fused SDPA"
    ref_seq, ref_logits = decode(False)
    scale = ref_logits[0].abs().max().item()
    assert (logits[0] - ref_logits[0]).abs().max().item() <= 0.02 * scale
    assert (seq == ref_seq).float().mean().item() >= 0.9


def gemma2_bf16(softcap, seed=0):
    from transformers import Gemma2Config, Gemma2ForCausalLM

    torch.manual_seed(seed)
    # Gemma 2's options: a sliding window (16 positions) on every other layer and, when given,
    # logit soft-capping; head_dim 128 with 4 query heads over 2 kv heads
    cfg = Gemma2Config(vocab_size=512, hidden_size=256, intermediate_size=512, num_hidden_layers=2,
                       num_attention_heads=4, num_key_value_heads=2, head_dim=128, max_position_embeddings=1024,
                       sliding_window=16, attn_logit_softcapping=softcap, final_logit_softcapping=None,
                       query_pre_attn_scalar=128, pad_token_id=0, eos_token_id=None, bos_token_id=1)
    return Gemma2ForCausalLM(cfg).to(torch.bfloat16).eval(), cfg


@pytest.mark.parametrize("softcap", [None, 20.0], ids=["window", "window_softcap"])
def test_paged_route_sliding_window_and_softcap_on_gpu(hip, monkeypatch, softcap):
    """The "barq_paged" route on a bf16 Gemma 2 on the GPU: full-attention layers decode through the
    page kernel, sliding-window layers past their window attend over the gathered K/V under the
    window mask transformers builds, soft-capped layers through the fp32 attention that applies
    the cap -- token by token against the same route with every call on the fp32 attention (the
    kernel and fused SDPA off): logits agree to bf16 rounding, greedy tokens agree."""
    pytest.importorskip("transformers")
    from barqtrain import create_paged_kv_cache
    from barqtrain_amd import attention
    from barqtrain_amd.paged import PagePool

    model, cfg = gemma2_bf16(softcap)
    model = model.to("cuda")
    attention.enable_paged_attention(model)
    prompt, new = 37, 20
    seq = torch.randint(2, 512, (2, prompt + new), generator=torch.Generator().manual_seed(9)).to("cuda")
    calls = []
    attend = PagePool.attend
    monkeypatch.setattr(PagePool, "attend", lambda self, *a, **k: calls.append(1) or attend(self, *a, **k))

    def run(reference: bool):
        if reference:
            monkeypatch.setattr(attention, "_KERNEL_MAX_ROWS", 0)
            monkeypatch.setattr(attention, "_sdpa_attention", lambda *a: None)
        cache = create_paged_kv_cache(model, max_batch_size=2, max_cache_len=prompt + new, page_size=16)
        steps = []
        with torch.no_grad():
            out = model(seq[:, :prompt], past_key_values=cache, use_cache=True)
            steps.append(out.logits[:, -1].float())
            for t in range(new - 1):
                out = model(seq[:, prompt + t:prompt + t + 1], past_key_values=cache, use_cache=True)
                steps.append(out.logits[:, -1].float())
        assert all(layer.pool.errors() == 0 for layer in cache.layers)
        return torch.stack(steps)

    routed = run(False)
    # the full-attention layer (every other one) runs the kernel when nothing caps its scores
    assert len(calls) == (0 if softcap else (new - 1) * cfg.num_hidden_layers // 2), len(calls)
    reference = run(True)
    scale = reference.abs().max().item()
    err = (routed - reference).abs().max().item()
    assert err <= 0.02 * scale, f"logits differ by {err} (scale {scale})"
    assert (routed.argmax(-1) == reference.argmax(-1)).float().mean().item() >= 0.9


def test_long_prefill_stays_within_memory(hip):
    """A 16k-token prefill of one row through the paged route: attention over the gathered K/V
    runs in fused SDPA (no [heads, T, S] score tensor: that would be 32 GiB in fp32); the last
    query rows match an fp32 attention computed for those rows alone."""
    from barqtrain_amd import attention
    from barqtrain_amd.kv_cache import BarqPagedKVCacheLayer

    T, Hkv, G, D = 16384, 8, 4, 128
    dev = torch.device("cuda", 0)
    gen = torch.Generator(device=dev).manual_seed(4)
    layer = BarqPagedKVCacheLayer(max_batch_size=1, max_cache_len=T, page_size=32)
    k = torch.randn((1, T, Hkv, D), generator=gen, device=dev).to(torch.bfloat16).transpose(1, 2)
    v = torch.randn((1, T, Hkv, D), generator=gen, device=dev).to(torch.bfloat16).transpose(1, 2)
    q = torch.randn((1, T, G * Hkv, D), generator=gen, device=dev).to(torch.bfloat16).transpose(1, 2)
    kk, vv = layer.update(k, v)
    torch.cuda.synchronize()
    torch.cuda.reset_peak_memory_stats()
    base = torch.cuda.memory_allocated()
    out = attention._gathered_attention(q, kk, vv, None, D ** -0.5)  # [1, T, Hq, D]
    torch.cuda.synchronize()
    assert torch.cuda.max_memory_allocated() - base < 2 * 2**30
    rows = 16
    qs = q[:, :, -rows:].float()
    sc = torch.matmul(qs, kk.float().repeat_interleave(G, 1).transpose(-1, -2).contiguous()) * D ** -0.5
    pos = torch.arange(T, device=dev)
    limit = T - rows + torch.arange(rows, device=dev)
    sc = sc.masked_fill(pos[None, :] > limit[:, None], float("-inf"))
    ref = torch.matmul(torch.softmax(sc, -1), vv.float().repeat_interleave(G, 1)).transpose(1, 2)
    err = (out[:, -rows:].float() - ref).abs().max().item()
    assert err <= 2.0 ** -7 * ref.abs().max().item() + 1e-3, err


def test_eager_step_planned_in_the_binding(hip):
    """PagePool.update / append on GPU pools plan in the binding (pool_step_): the same outputs
    and host shadow as the checked path, and every refusal raises what the checked path raises,
    changing nothing (free pages, capacity, dtype, batch); empty calls still gather."""
    from barqtrain_amd.paged import PagedKVCapacityError, PagedKVPoolExhausted, PagePool

    H, D, P = 2, 64, 16
    pool = PagePool(max_batch=3, max_blocks=4, page_size=P, kv_heads=H, head_dim=D, dtype=torch.bfloat16,
                    device="cuda", num_pages=9)
    oracle = DenseLayerOracle(3, 64, P)
    gen = torch.Generator().manual_seed(11)
    for t in (20, 1, 13):
        k, v = hf_layout(3, H, t, D, torch.bfloat16, gen), hf_layout(3, H, t, D, torch.bfloat16, gen)
        gk, gv = pool.update(k.cuda(), v.cuda())
        ok, ov = oracle.update(to_bits(k), to_bits(v))
        assert_bits(gk, ok, f"K after {t}")
        assert_bits(gv, ov, f"V after {t}")
    k = hf_layout(2, H, 3, D, torch.bfloat16, gen)
    pool.append(k.cuda(), k.cuda())
    oracle.append(to_bits(k), to_bits(k))
    assert pool.lens.tolist() == [37, 37, 34] and pool.hw.tolist() == [37, 37, 34]
    assert pool.free_count == int(pool.ctrl[0].item()) == 9 - 9
    gk, _ = pool.gather(2)
    assert_bits(gk, oracle.current_tensors()[0], "K after append")
    state = (pool.lens.copy(), pool.hw.copy(), pool.free_count)
    one = torch.zeros((1, H, 1, D), dtype=torch.bfloat16, device="cuda")
    with pytest.raises(PagedKVPoolExhausted):  # row 2 at 34 + 15 crosses into a fourth block
        pool.update(torch.zeros((3, H, 15, D), dtype=torch.bfloat16, device="cuda"),
                    torch.zeros((3, H, 15, D), dtype=torch.bfloat16, device="cuda"))
    with pytest.raises(PagedKVCapacityError):
        pool.update(one, one, max_length=37)
    with pytest.raises(RuntimeError):  # the binding's dtype check, as before the fast path
        pool.update(one.float(), one.float())
    with pytest.raises(ValueError):
        big = torch.zeros((4, H, 1, D), dtype=torch.bfloat16, device="cuda")
        pool.append(big, big)
    assert (pool.lens.copy(), pool.hw.copy(), pool.free_count)[2] == state[2]
    assert np.array_equal(pool.lens, state[0]) and np.array_equal(pool.hw, state[1])
    empty = torch.zeros((3, H, 0, D), dtype=torch.bfloat16, device="cuda")
    gk, gv = pool.update(empty, empty)
    ok, _ = oracle.update(to_bits(empty.cpu()), to_bits(empty.cpu()))
    assert gk.shape == (3, H, 37, D)
    assert_bits(gk, ok, "K of an empty update")
