"""Mirror a paged cache's operations into per-layer QuantLayerOracles while a model runs.

``shadow(cache, monkeypatch)`` wraps every layer's ``update`` (each returned K/V is compared with
the oracle's, bit for bit, after feeding the oracle the same input bits), ``crop``, the per-layer
selections and the all-layer selection (``kv_cache.select_rows_layers``), so a ``generate()``
with beam search checks the quantised cache against the oracle at every step and every beam
reordering.  Returns the list of per-layer counters {"updates", "selections"}.
"""

from __future__ import annotations

import numpy as np

from kvgen import to_bits
from oracle.kv_quant_oracle import QuantLayerOracle

DT = {"torch.bfloat16": "bf16", "torch.float16": "f16", "torch.float32": "f32"}


def shadow(cache, monkeypatch):
    from barqtrain_amd import kv_cache

    stats = []
    by_pool = {}

    def oracle_of(layer):
        o = getattr(layer, "_shadow_oracle", None)
        if o is None:  # created at the layer's first append, when its geometry is known
            o = QuantLayerOracle(layer.max_batch_size, layer.max_cache_len, layer.page_size,
                                 layer.residual_window, DT[str(layer.dtype)])
            layer._shadow_oracle = o
        return o

    for i, layer in enumerate(cache.layers):
        counts = {"updates": 0, "selections": 0}
        stats.append(counts)

        def update(key_states, value_states, *args, _layer=layer, _f=layer.update, _c=counts, **kwargs):
            out = _f(key_states, value_states, *args, **kwargs)
            o = oracle_of(_layer)
            by_pool[id(_layer.pool)] = o
            ok, ov = o.update(to_bits(key_states.detach().cpu()), to_bits(value_states.detach().cpu()))
            gk, gv = to_bits(out[0].detach().cpu()), to_bits(out[1].detach().cpu())
            assert np.array_equal(gk, ok) and np.array_equal(gv, ov), f"update {_c['updates']}"
            _c["updates"] += 1
            return out

        def crop(max_length, _layer=layer, _f=layer.crop):
            _f(max_length)
            oracle_of(_layer).crop(max_length)

        def select(rows, _layer=layer, _f=layer._select_rows, _c=counts):
            _f(rows)
            oracle_of(_layer).batch_select_indices(rows)
            _c["selections"] += 1

        monkeypatch.setattr(layer, "update", update)
        monkeypatch.setattr(layer, "crop", crop)
        monkeypatch.setattr(layer, "_select_rows", select)

    def select_all(pools, rows, _f=kv_cache.select_rows_layers):
        _f(pools, rows)
        for p in pools:
            by_pool[id(p)].batch_select_indices([int(r) for r in rows])
        for c in stats:
            c["selections"] += 1

    monkeypatch.setattr(kv_cache, "select_rows_layers", select_all)
    return stats
