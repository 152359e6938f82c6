"""miso_amd: MI355X (gfx950) gated GQA softmax attention -- the decode (split-K + LSE merge) and
causal prefill (f16 MFMA flash attention) path of the miso Qwen3.5-MoE engine, as a C++ header
API (miso_amd/kernels) and a C ABI shared library (include/miso_attn.h, miso_amd/lib).

Import the operators with `from miso_amd import attention`; it loads the built library and fails
loudly if it is missing.
"""

__all__ = ["attention", "build"]
