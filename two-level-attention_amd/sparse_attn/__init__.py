"""MI355X-native drop-in for the NFA decode path of ``sparse_attn``.

Same module paths and entry points as the reference package
(Chosen-David/two-level-attention ``sparse_attn``) for the two-level sparse
decode layer: ``indexer.nfa_layer_batch_selector.select_topk_for_layer_batched``,
``ops.paged_region_kernels.sparse_paged_attention_gather`` and the
graph-ready paged cache.  The device work runs in ``lib/libnfa_hip.so``
(hand-written HIP for gfx950) through a C ABI.
"""
