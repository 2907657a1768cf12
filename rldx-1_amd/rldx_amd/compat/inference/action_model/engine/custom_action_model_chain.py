"""Mirror of rldx/inference/action_model/engine/custom_action_model_chain.py:
the action head chain built from a GraphSafeActionModel, served by the
rldx_amd action head (vlln, state encoder, RTC trained-mode prefix, per step
action encoder + MSAT + decoder + Euler update as one hipGraph) behind an
ActionHeadDispatcher.  A batch of B robots runs on a graph for B (up to the
dispatcher's max_batch); other calls (a larger batch, a missing prefix) go to
the GraphSafeActionModel's own forward, which computes the same actions
(graph_safe_action_model.py:171-315).
torch.compile is not used: the captured graph is what compilation buys the
reference (one launch sequence per call)."""

from __future__ import annotations

import time

import torch

from rldx_amd.rldx_msat import ActionHeadDispatcher


class CustomActionHeadChain(torch.nn.Module):
    """CustomActionHeadChain (custom_action_model_chain.py:23-171): same
    constructor and forward signature; the baked values (position embedding,
    per-step time embeddings and time tokens) are computed from
    gs_action_model the same way when the head is built."""

    def __init__(self, gs_action_model, device, dtype=torch.bfloat16):
        super().__init__()
        if dtype != torch.bfloat16:
            raise ValueError("the rldx_amd action head computes in bfloat16")
        self.action_horizon = gs_action_model.action_horizon
        self.action_dim = gs_action_model.action_dim
        self.num_inference_timesteps = gs_action_model.num_inference_timesteps
        self.dt = gs_action_model.dt
        self.prefix_len = getattr(gs_action_model, "prefix_len", 0)
        self.device = torch.device(device)
        self.dispatcher = ActionHeadDispatcher(gs_action_model, graph=True)
        self.dispatcher.build()

    def forward(self, vl_embs, state, embodiment_id, init_noise=None, prefix_actions=None, **kwargs):
        return self.dispatcher(vl_embs, state, embodiment_id, init_noise=init_noise, prefix_actions=prefix_actions)


def build_custom_action_model_chain(action_head_model, device, dtype=torch.bfloat16):
    """custom_action_model_chain.py:174-176."""
    return CustomActionHeadChain(action_head_model, device=device, dtype=dtype).eval()


def compile_custom_action_model_chain(chain, sample_inputs, compile_mode="max-autotune", fullgraph=True):
    """custom_action_model_chain.py:179-198: returns (chain, seconds) after one
    call on sample_inputs (vl_embs, state, embodiment_id, init_noise); the head's
    graph was captured at build, so nothing is compiled."""
    vl_embs, state, embodiment_id, init_noise = sample_inputs
    t0 = time.time()
    with torch.no_grad():
        chain(vl_embs, state, embodiment_id, init_noise=init_noise)
    torch.cuda.synchronize()
    return chain, time.time() - t0
