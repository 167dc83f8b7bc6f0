"""Drop-in replacement for the reference's lact_moe_triton package
(uttt_llm/flame/custom_models/uttt_moe/lact_moe_triton/): the same module and
function names, backed by the gfx950 HIP kernels of libuttt_hip.so.  Kernel
modules are imported directly from the subpackage as needed."""
