#!/usr/bin/env python3
"""Writes tests/golden/inkling_moe.npz: golden vectors for the MoE router and
layer composition from the third-party transformers implementation of the
Inkling sparse MoE (transformers 5.15.0, models/inkling/modeling_inkling.py:
InklingTopkRouter, InklingExperts, InklingSharedExperts, InklingMoE), which
restates the same specification the reference follows
(docs/architecture-notes.md:340-474 of the reference; src/sepia.c:1329-1470).

The reference's own router/MoE code is static inside src/sepia.c and its model
test needs weights that are not in the repository, so these vectors are the
independent pin for route selection, mixing weights and the order of the
shared/routed combination. The module runs in float64 on fp32-representable
inputs, so the expected outputs carry no fp32 rounding of their own.

Shapes are tiny (hidden 32, moe_intermediate 16, 16 routed + 2 shared
experts, top-6, 8 tokens); gate and up are stored as separate tensors (the
module's gate_up_proj is [gate rows; up rows], not interleaved).

Run from the repository root:  python tests/golden/make_inkling_moe.py
"""
import os
import types

import numpy as np
import torch

from transformers.models.inkling import modeling_inkling as mi

H, I, NR, NS, TOPK, TOKENS = 32, 16, 16, 2, 6, 8
ROUTE_SCALE, GLOBAL_SCALE = 8.0, 0.75


def f32(a):
    return np.asarray(a, dtype=np.float32)


def main():
    rng = np.random.default_rng(20260101)
    router_w = f32(rng.standard_normal((NR + NS, H)) * 0.3)
    router_b = f32(rng.uniform(-0.1, 0.1, NR))
    gate = f32(rng.standard_normal((NR, I, H)) * 0.2)
    up = f32(rng.standard_normal((NR, I, H)) * 0.2)
    down = f32(rng.standard_normal((NR, H, I)) * 0.2)
    s_gate = f32(rng.standard_normal((NS, I, H)) * 0.2)
    s_up = f32(rng.standard_normal((NS, I, H)) * 0.2)
    s_down = f32(rng.standard_normal((NS, H, I)) * 0.2)
    x = f32(rng.standard_normal((TOKENS, H)))

    cfg = types.SimpleNamespace(n_routed_experts=NR, n_shared_experts=NS, hidden_size=H, route_scale=ROUTE_SCALE,
                                num_experts_per_tok=TOPK, moe_intermediate_size=I, hidden_act="silu",
                                _experts_implementation=None)
    m = mi.InklingMoE(cfg).double()
    with torch.no_grad():
        m.gate.weight.copy_(torch.from_numpy(router_w.astype(np.float64)))
        m.gate.e_score_correction_bias.copy_(torch.from_numpy(router_b.astype(np.float64)))
        m.gate.global_scale.fill_(GLOBAL_SCALE)
        m.experts.gate_up_proj.copy_(torch.from_numpy(np.concatenate([gate, up], axis=1).astype(np.float64)))
        m.experts.down_proj.copy_(torch.from_numpy(down.astype(np.float64)))
        m.shared_experts.gate_proj.copy_(torch.from_numpy(s_gate.astype(np.float64)))
        m.shared_experts.up_proj.copy_(torch.from_numpy(s_up.astype(np.float64)))
        m.shared_experts.down_proj.copy_(torch.from_numpy(s_down.astype(np.float64)))
        xt = torch.from_numpy(x.astype(np.float64))
        logits, topk_w, topk_idx, gammas = m.gate(xt)
        y = m(xt.view(1, TOKENS, H)).view(TOKENS, H)
    # the router returns the selection unsorted; store it sorted by expert id
    # with its weights permuted alike (the set and the pairing are what matter)
    idx = topk_idx.numpy().astype(np.int32)
    w = topk_w.numpy()
    order = np.argsort(idx, axis=1)
    idx = np.take_along_axis(idx, order, axis=1)
    w = np.take_along_axis(w, order, axis=1)
    out = os.path.join(os.path.dirname(os.path.abspath(__file__)), "inkling_moe.npz")
    np.savez_compressed(out, x=x, router_w=router_w, router_b=router_b, gate=gate, up=up, down=down,
                        s_gate=s_gate, s_up=s_up, s_down=s_down,
                        route_scale=np.float64(ROUTE_SCALE), global_scale=np.float64(GLOBAL_SCALE),
                        topk=np.int32(TOPK), logits=logits.numpy(), idx=idx, w_routed=w,
                        gammas=gammas.numpy(), y=y.numpy())
    print("wrote", out, os.path.getsize(out), "bytes")


if __name__ == "__main__":
    main()
