"""exactinfer_amd — MI355X (gfx950) Qwen3 attention hot path: QK-norm + RoPE, KV append,
split-K decode and fp32-MFMA causal prefill behind the C ABI of include/ei_attn.h."""

__version__ = "0.1.0"
