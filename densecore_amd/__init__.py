"""densecore_amd: DenseCore's scaled-dot-product-attention path, MI355X-native.

Hand-written HIP kernels for gfx950 (``csrc/``) behind the C ABI in ``include/dc_attn.h``
(``libdcattn.so``), with a Python layer that mirrors the reference's boundary
(``_native._flash_attention`` / ``_flash_attention_backward``) and its public
``functional.scaled_dot_product_attention``.
"""
from . import functional  # noqa: F401
from . import nn, random  # noqa: F401
from ._native import _flash_attention, _flash_attention_backward, _flash_decode, consistent_scores  # noqa: F401

__all__ = ["functional", "nn", "random", "_flash_attention", "_flash_attention_backward", "_flash_decode",
           "consistent_scores"]
