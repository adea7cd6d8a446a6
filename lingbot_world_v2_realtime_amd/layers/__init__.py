"""The DiT-layer surface of the quantized attention path (mirrors lingbot/layers)."""
