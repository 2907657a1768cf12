"""Mirror of rldx/inference/backbone/llm/engine/kernels/ on the rldx_amd gfx950 kernels
(the reference's launcher names and signatures)."""
