"""torch.library.opcheck of every ``fastdecisions::`` op.

The reference runs its ops inside ``torch.compile`` (ref: src/decider/engine.py:106-108;
ref: experiments/native_gqa/bench_native_gqa_model.py:116-121), where Dynamo traces them
through their ``register_fake`` implementations (ref: src/decider/packed_conv.py:17-21):
the fake's shapes, strides and dtypes must be the real op's.  opcheck runs the op for
real and under fake tensors and compares them (``test_faketensor``), checks the schema
against the op's behaviour (``test_schema``: no input mutated, no output aliasing an
input), that calling it with grad-requiring inputs is refused rather than silently
differentiated (``test_autograd_registration``), and that it traces under AOT dispatch
with dynamic shapes (``test_aot_dispatch_dynamic``).  Inputs are small decider-shaped
tensors in the layouts the model passes (strided views of combined projections).
"""
from __future__ import annotations

import pytest
import torch

from helpers import announce

pytestmark = pytest.mark.gpu


def _r(*shape, scale=1.0, dtype=torch.bfloat16, seed=0):
    g = torch.Generator().manual_seed(seed)
    return (torch.randn(shape, generator=g) * scale).to(dtype).cuda()


def _cases():
    import fastdecisions_amd.combined_gates  # noqa: F401  (registers the ops)
    import fastdecisions_amd.gated_delta  # noqa: F401
    import fastdecisions_amd.layer_fusions  # noqa: F401
    import fastdecisions_amd.native_gqa  # noqa: F401
    import fastdecisions_amd.packed_conv  # noqa: F401
    import fastdecisions_amd.persistent_residual_rms  # noqa: F401
    ops = torch.ops.fastdecisions
    T, H, D = 96, 16, 128
    cu = torch.tensor([0, 40, 40, 96], dtype=torch.int32, device="cuda")
    # attention: q | gate per head and k, v from one projection (the fused layer's views)
    proj = _r(1, T, 4 * H * D // 2 + 2 * 4 * D, seed=1)
    qg = proj[..., :2 * 16 * D].view(1, T, 16, 2 * D)
    q, gate = qg[..., :D].transpose(1, 2), qg[..., D:].transpose(1, 2)
    k = proj[..., 2 * 16 * D:2 * 16 * D + 4 * D].view(1, T, 4, D).transpose(1, 2)
    v = proj[..., 2 * 16 * D + 4 * D:].view(1, T, 4, D).transpose(1, 2)
    cos, sin = _r(1, T, 32, seed=2), _r(1, T, 32, seed=3)
    wq, wk = _r(D, scale=0.02, seed=4), _r(D, scale=0.02, seed=5)
    # Gated-DeltaNet: conv input q|k|v, its weight, gates, z
    x = _r(1, T, 3 * H * D, seed=6)
    conv_w = _r(3 * H * D, 1, 4, scale=0.25, seed=7)
    hidden = _r(1, T, 2048, seed=8)
    gate_w = _r(2 * H, 2048, scale=0.02, seed=9)
    a_log = torch.empty(H).uniform_(1, 16).log().cuda()
    dt_bias = torch.ones(H, device="cuda")
    ab = _r(1, T, 2 * H, seed=10)
    dq, dk, dv = (_r(1, T, H, D, seed=11 + i) for i in range(3))
    g = -torch.rand((1, T, H), generator=torch.Generator().manual_seed(14)).cuda()
    beta = torch.rand((1, T, H), generator=torch.Generator().manual_seed(15)).to(torch.bfloat16).cuda()
    z = _r(1, T, H, D, seed=16)
    norm_w = 1.0 + _r(D, scale=0.02, seed=17)
    # residual stream and MLP
    a, b, w = _r(2, T, 2048, seed=18), _r(2, T, 2048, seed=19), _r(2048, scale=0.02, seed=20)
    gu = _r(2, T, 2 * 512, seed=21)
    gu2 = _r(2, T, 2 * 256, seed=22)
    return [
        ("native_gqa", ops.native_gqa, (q, k, v)),
        ("native_gqa_varlen", ops.native_gqa_varlen, (q, k, v, cu, 56)),
        ("native_gqa_gated", ops.native_gqa_gated, (q, k, v, gate, None, T)),
        ("native_gqa_gated varlen", ops.native_gqa_gated, (q, k, v, gate, cu, 56)),
        ("attn_prologue", ops.attn_prologue, (q.transpose(1, 2), k.transpose(1, 2), wq, wk, cos, sin, 1e-6)),
        ("packed_conv", ops.packed_conv, (x, conv_w)),
        ("packed_conv_varlen", ops.packed_conv_varlen, (x, conv_w, cu)),
        ("packed_conv_gates", ops.packed_conv_gates, (x, conv_w, hidden, gate_w, a_log, dt_bias, None)),
        ("packed_conv_gates varlen", ops.packed_conv_gates, (x, conv_w, hidden, gate_w, a_log, dt_bias, cu)),
        ("gate_transform", ops.gate_transform, (ab[..., :H], ab[..., H:], a_log, dt_bias)),
        ("gate_proj", ops.gate_proj, (hidden, gate_w, a_log, dt_bias)),
        ("unpack_gate", ops.unpack_gate, (ab, a_log, dt_bias)),
        ("gated_delta_rule", ops.gated_delta_rule, (dq, dk, dv, g, beta, None)),
        ("gated_delta_rule varlen", ops.gated_delta_rule, (dq, dk, dv, g, beta, cu)),
        ("gated_delta_rule_norm", ops.gated_delta_rule_norm, (dq, dk, dv, g, beta, z, norm_w, 1e-6, None)),
        ("residual_rms", ops.residual_rms, (a, b, w)),
        ("fused_add_rms_norm", ops.fused_add_rms_norm, (a, b, w, 1e-6)),
        ("rms_norm", ops.rms_norm, (a, w, 1e-6)),
        ("gated_rms_norm", ops.gated_rms_norm, (dv.reshape(-1, D), z, norm_w, 1e-6)),
        ("silu_mul", ops.silu_mul, (gu,)),
        ("silu_mul_split", ops.silu_mul_split, (gu, gu2)),
    ]


def test_every_op_is_covered():
    """Every op registered under ``fastdecisions::`` has a case below."""
    names = {name.split()[0] for name, _, _ in _cases()}
    registered = {n for n in torch._C._dispatch_get_all_op_names() if n.startswith("fastdecisions::")}
    assert registered == {f"fastdecisions::{n}" for n in names}, registered ^ {f"fastdecisions::{n}" for n in names}


@pytest.mark.parametrize("index", range(21))
def test_opcheck(index):
    name, op, args = _cases()[index]
    announce(f"opcheck fastdecisions::{name}")
    torch.library.opcheck(op, args)
    torch.cuda.synchronize()
