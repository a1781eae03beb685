"""AWQ W4A16 linear layer for MI355X: ``awq`` (W4Linear and its helpers), ``w4_hip`` (the C-ABI
library and split-K workspace), ``linear`` (make_linear / finalize_quantized)."""
