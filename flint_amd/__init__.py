"""flint_amd — MI355X-native batch-1 int4 decode engine (HIP kernels behind a C ABI).

Modules: _lib (ctypes C-ABI binding), quantize (int4 quantise / dequantise / GEMV, gpt-fast's
WeightOnlyInt4Linear), synth (ModelArgs + seeded synthetic weights), model (packed model +
Transformer handle), generate (prefill / decode_one_token / decode_n_tokens / generate),
spec (speculative chain / tree loops over verify, KV compaction), checkpoint (HF / gpt-fast /
packed int4 files on disk).
"""
__version__ = "0.1.0"
