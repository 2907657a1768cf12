"""Mirror of rldx/inference/action_model/double_stream/engine/kernels/ on the rldx_amd gfx950 kernels
(the reference's launcher names and signatures)."""
