"""Mirror of rldx/inference/memory/engine/kernels/ on the rldx_amd gfx950 kernels
(the reference's launcher names and signatures)."""
