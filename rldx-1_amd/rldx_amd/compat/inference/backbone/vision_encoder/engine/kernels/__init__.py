"""Mirror of rldx/inference/backbone/vision_encoder/engine/kernels/ on the rldx_amd gfx950 kernels
(the reference's launcher names and signatures)."""
