"""Builds one seeded random-init model on the host (CPU oracle generator) and
hands the same tensors to the oracle and to a GPU anehip.Model."""
import numpy as np

import anehip
import oracle

SMALL = dict(dim=256, hidden_dim=512, n_layers=4, n_heads=4, n_kv_heads=1, head_dim=256, vocab_size=1000,
             ssm_state_size=128, ssm_conv_kernel=4, ssm_group_count=2)
# A model whose batch > 1 projections all run on the x-stationary GEMM with
# K splits (the small model's 256-wide matrices take a single split).
MID = dict(dim=512, hidden_dim=1024, n_layers=4, n_heads=4, n_kv_heads=1, head_dim=256, vocab_size=1000,
           ssm_state_size=128, ssm_conv_kernel=4, ssm_group_count=4)

# A model 2304 wide (18 DeltaNet heads, 9 panels per row): its batch-1 ssm_out
# would need 9 K splits, one per head pair, beyond the 8 partial slices a
# consumer adds, so its batch-1 step runs the DeltaNet step as its own kernel
# (deltanet_step_kernel) and the ssm_out GEMV's gated-norm prologue commits
# the q / k conv windows, instead of the step fused into ssm_out.
WIDE = dict(dim=2304, hidden_dim=512, n_layers=4, n_heads=8, n_kv_heads=2, head_dim=256, vocab_size=1000,
            ssm_state_size=128, ssm_conv_kernel=4, ssm_group_count=18)


class HostModel:
    def __init__(self, spec: "anehip.Spec", seed: int = 1, ggml_type: int = 8):
        self.spec, self.ggml_type = spec, ggml_type
        self.tensors = {}
        for layer in [-1] + list(range(spec.n_layers)):
            for kind, (rows, cols, quant) in spec.shapes(layer).items():
                st = (layer + 1) * 64 + kind
                if quant:
                    arr = oracle.gen_quant(ggml_type, seed, st, rows, cols, std=anehip.WEIGHT_STD)
                else:
                    dist, a, b = anehip.F32_RECIPE[kind]
                    arr = (oracle.normal(seed, st, rows * cols, mean=a, std=b) if dist == 0
                           else oracle.uniform(seed, st, rows * cols, lo=a, hi=b))
                self.tensors[(layer, kind)] = (arr, rows, cols, quant)
        s = spec
        self.om = oracle.OracleModel(s.dim, s.hidden_dim, s.n_layers, s.n_heads, s.n_kv_heads, s.head_dim,
                                     s.vocab_size, s.ssm_state_size, s.ssm_conv_kernel, s.ssm_group_count,
                                     s.rope_freq_base, s.rms_norm_eps, s.layer_types)
        for (layer, kind), (arr, rows, cols, quant) in self.tensors.items():
            if quant:
                self.om.set_quant(layer, kind, arr, rows, cols, ggml_type)
            else:
                self.om.set_f32(layer, kind, arr)

    def upload(self, gm: "anehip.Model"):
        for (layer, kind), (arr, rows, cols, quant) in self.tensors.items():
            if quant:
                gm.upload_quant(layer, kind, arr, rows, cols, self.ggml_type)
            else:
                gm.upload_f32(layer, kind, arr)

    def seq(self, max_seq: int) -> "oracle.OracleSeq":
        return oracle.OracleSeq(self.om, max_seq, kv_f16=True)


def copy_state_to_oracle(gm: "anehip.Model", oseq: "oracle.OracleSeq", b: int):
    """Copies sequence b's GPU state (conv windows, S, KV, pos) into an oracle sequence."""
    s = gm.spec
    for l in range(s.n_layers):
        if s.layer_types[l] == anehip.LAYER_DELTANET:
            conv = gm.get_state(l, 0, b)
            S = gm.get_state(l, 1, b)
            oseq.view(l, 0, conv.size, np.float32)[:] = conv
            oseq.view(l, 1, S.size, np.float32)[:] = S
        else:
            for which in (2, 3):
                kv = gm.get_state(l, which, b)
                oseq.view(l, which, kv.size, np.uint16)[:] = kv
    oseq.pos = gm.get_pos(b)
