"""Adapter package named like flash-linear-attention ("fla") so that
transformers' Qwen3.5 gated-delta-net layers run on the gfx950 HIP ops.

transformers resolves ``fla.ops.gated_delta_rule.chunk_gated_delta_rule`` and
``...recurrent_gated_delta_rule`` when ``fla`` is importable
(transformers/integrations/hub_kernels.py:65-67,764-801; the call sites are
models/qwen3_5/modeling_qwen3_5.py:248,330,505-529).  Put the directory that
holds this package (``qwen-drive-edge-orin_amd/hf``) on ``sys.path`` before
transformers imports the model to opt in.  Only the two gated-delta-rule entry
points exist here; nothing else of the real package is provided.
"""

from .ops.gated_delta_rule import chunk_gated_delta_rule, recurrent_gated_delta_rule  # noqa: E402,F401
