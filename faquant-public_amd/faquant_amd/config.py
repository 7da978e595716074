"""Attention-path configuration constants (reference: src/faquant/config.py:15-24, 50-51)."""

PV_NORMALIZER_MODES = ("unquantized", "quantized_same")
"""Softmax denominator source: the raw tile probabilities (``unquantized``) or
the row sum of the same quantized P that feeds PV (``quantized_same``,
P-Reordering)."""

DEFAULT_QUERY_CHUNK = 256
DEFAULT_KEY_CHUNK = 128
