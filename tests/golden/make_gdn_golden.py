"""Writes tests/golden/gdn_transformers.npz: golden vectors for the gated delta rule from an
independent implementation, transformers' qwen3_5 `torch_recurrent_gated_delta_rule`
(third-party text installed in this container; not the reference, which is never imported).

Run from the repo root: python tests/golden/make_gdn_golden.py
The inputs are seeded; the file holds inputs and outputs only (data, no code).
"""

import os

import numpy as np
import torch
from transformers.models.qwen3_5.modeling_qwen3_5 import torch_recurrent_gated_delta_rule

OUT = os.path.join(os.path.dirname(os.path.abspath(__file__)), "gdn_transformers.npz")


def main():
    g = torch.Generator().manual_seed(0)
    T, H, Dk, Dv = 5, 3, 16, 8
    q = torch.randn((1, T, H, Dk), generator=g, dtype=torch.float64)
    k = torch.randn((1, T, H, Dk), generator=g, dtype=torch.float64)
    v = torch.randn((1, T, H, Dv), generator=g, dtype=torch.float64)
    a = torch.randn((1, T, H), generator=g, dtype=torch.float64)
    b = torch.randn((1, T, H), generator=g, dtype=torch.float64)
    A_log = torch.log(torch.rand((H,), generator=g, dtype=torch.float64) * 15 + 1)
    dt_bias = torch.rand((H,), generator=g, dtype=torch.float64) * 2 - 1
    S0 = torch.randn((1, H, Dk, Dv), generator=g, dtype=torch.float64) * 0.5
    # the gate formula of transformers' Qwen3_5GatedDeltaNet.forward
    gl = -A_log.exp() * torch.nn.functional.softplus(a + dt_bias)
    beta = b.sigmoid()
    y, S = torch_recurrent_gated_delta_rule(q, k, v, g=gl, beta=beta, initial_state=S0, output_final_state=True,
                                            use_qk_l2norm_in_kernel=True)
    # per-token states: run prefixes
    states = []
    for t in range(1, T + 1):
        _, St = torch_recurrent_gated_delta_rule(q[:, :t], k[:, :t], v[:, :t], g=gl[:, :t], beta=beta[:, :t],
                                                 initial_state=S0, output_final_state=True,
                                                 use_qk_l2norm_in_kernel=True)
        states.append(St[0].numpy())
    np.savez(OUT, q=q[0].numpy(), k=k[0].numpy(), v=v[0].numpy(), a=a[0].numpy(), b=b[0].numpy(),
             A_log=A_log.numpy(), dt_bias=dt_bias.numpy(), S0_kv=S0[0].numpy(), y=y[0].numpy(),
             S_final_kv=S[0].numpy(), states_kv=np.stack(states))
    print("wrote", OUT)


if __name__ == "__main__":
    main()
