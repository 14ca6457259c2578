"""Quantized-weight formats and linears on MI355X (the API of ``scratch_llm.quant``)."""
