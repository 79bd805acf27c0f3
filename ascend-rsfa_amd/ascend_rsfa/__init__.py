"""ascend_rsfa for MI355X: FlashAttention-2 forward on gfx950.

Drop-in for the reference package's import path
``ascend_rsfa.flash_attention_forward`` (reference ascend_rsfa/__init__.py:1-3).
"""

__version__ = "0.1.0"
