"""Mirror of rldx/inference/action_model/engine/custom_expanded_action_model_chain.py:
the all-add-ons action head chain (with the physics head) built from a
GraphSafeActionModel, served by the rldx_amd action head with its P stream
(history tokens encoded once; per step the future physics state at the step's
time, MSAT over [VL | SA | P], action and physics decoders, both Euler updates)
as one hipGraph behind an ActionHeadDispatcher.  A batch of B robots runs on a
graph for B (up to the dispatcher's max_batch); other calls go to the
GraphSafeActionModel's own forward."""

from __future__ import annotations

import time

import torch

from rldx_amd.rldx_msat import ActionHeadDispatcher


class CustomExpandedActionHeadChain(torch.nn.Module):
    """CustomExpandedActionHeadChain (custom_expanded_action_model_chain.py:19-213)."""

    def __init__(self, gs_action_model, device, dtype=torch.bfloat16):
        super().__init__()
        if dtype != torch.bfloat16:
            raise ValueError("the rldx_amd action head computes in bfloat16")
        self.action_horizon = gs_action_model.action_horizon
        self.action_dim = gs_action_model.action_dim
        self.num_inference_timesteps = gs_action_model.num_inference_timesteps
        self.dt = gs_action_model.dt
        self.prefix_len = getattr(gs_action_model, "prefix_len", 0)
        self.physics_hist_len = gs_action_model.physics_hist_len
        self.physics_fut_len = gs_action_model.physics_fut_len
        self.physics_dim = gs_action_model.physics_dim
        self.device = torch.device(device)
        self.dispatcher = ActionHeadDispatcher(gs_action_model, graph=True)
        self.dispatcher.build()

    def forward(self, vl_embs, state, embodiment_id, init_noise=None, physics_hist=None, physics_init_noise=None,
                prefix_actions=None):
        return self.dispatcher(vl_embs, state, embodiment_id, init_noise=init_noise, physics_hist=physics_hist,
                               physics_init_noise=physics_init_noise, prefix_actions=prefix_actions)


def build_custom_expanded_action_model_chain(action_head_model, device, dtype=torch.bfloat16):
    """custom_expanded_action_model_chain.py:216-218."""
    return CustomExpandedActionHeadChain(action_head_model, device=device, dtype=dtype).eval()


def compile_custom_expanded_action_model_chain(chain, sample_inputs, compile_mode="max-autotune", fullgraph=True):
    """custom_expanded_action_model_chain.py:221-245: returns (chain, seconds)
    after one call on sample_inputs (vl_embs, state, embodiment_id, init_noise,
    physics_hist, physics_init_noise); nothing is compiled."""
    vl_embs, state, embodiment_id, init_noise, physics_hist, physics_init_noise = sample_inputs
    t0 = time.time()
    with torch.no_grad():
        chain(vl_embs, state, embodiment_id, init_noise=init_noise, physics_hist=physics_hist,
              physics_init_noise=physics_init_noise)
    torch.cuda.synchronize()
    return chain, time.time() - t0
