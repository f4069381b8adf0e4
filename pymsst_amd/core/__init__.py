"""Restated stock modules of the RoFormer training path (the modules the fused kernels replace).

The reference (baicai-1145/pymsst) patches modules of its external model library
pymss-core 0.1.4, which is not available here.  This package restates those
modules in plain PyTorch from the public BS-RoFormer / Mel-band RoFormer
architecture, with the attribute and method names the reference's patch layer
binds to (``src/pymsst/training/fused_roformer.py:256-873``):

* ``bands``: ``BandSplit`` (``_forward_grouped``, ``_get_group_params``,
  ``_dim_offsets``, ``_dim_groups``), ``MaskEstimator``
  (``_forward_layer_grouped_mlp``, ``_layer_grouping_plan``, ...),
  ``grouped_linear``, ``inference_tanh``;
* ``transformer``: ``RMSNorm``, ``Attention``, ``FeedForward``, ``Transformer``,
  ``apply_rotary_emb_fast``, ``qkv_to_bnhd``, ``rotate_qk_fast_bnhd``;
* ``common``: ``RoformerRuntimeMixin`` (``_estimate_masks``);
* ``bs_roformer`` / ``mel_band_roformer``: the two model families.

These run on stock PyTorch (CPU or GPU).  They are the "stock" side of every
fused-vs-stock parity check and of the stock-vs-fused train-step benchmark.
"""
