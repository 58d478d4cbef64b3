"""pico_hip: MI355X (gfx950) decode path for GGUF Q4_K_M Qwen2-style models.

Host side (this package) mirrors the reference pico-engine's Python surface -- ``gguf``,
``dequant``, ``kernels``, ``model``, ``engine``, ``sampler``, ``tokenizer`` -- and drives
hand-written HIP kernels in ``libpico_hip.so`` through the C ABI of include/pico_hip.h.
Submodules that launch kernels import the library eagerly and raise if it is not built.
"""

__all__ = ["gguf", "dequant", "quantize", "synth", "kernels", "model", "engine", "sampler",
           "tokenizer"]
__version__ = "0.1.0"
