"""witchcraft_amd -- MI355X-native (gfx950) `t5-hip` backend for Witchcraft's XTR-T5 encoder.

Product: libt5hip.so (HIP kernels + the C ABI of include/t5hip.h), driven from C/C++/Rust
callers.  Python pieces: `encoder` (ctypes face of the C ABI, loads libt5hip.so and fails
if it is not built), `synth` / `quantize` / `gguf` (model-building tools).
"""

__all__ = ["encoder", "synth", "quantize", "gguf"]
