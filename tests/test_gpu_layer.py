"""Configuration 3: one 27B-shaped decode layer + Q6_K lm_head through the
HIP path, against the CPU oracle's composition of the same step. The greedy
token must be identical (sampling/root.zig:226-239); logits are also checked
normwise (2e-3). The CPU side (oracle/layer_oracle.py) follows the reference's
operations: matvecs with F64 accumulation (cpu/root.zig:112-165) and
silu(x) = f32(x * logistic(x)) in F64 (cpu/vector.zig:178-181)."""
import numpy as np
import pytest

import nuclis_amd as nq
from nuclis_amd import layer as L
from nuclis_amd.synth import gaussian
from oracle import layer_oracle
from oracle import oracle as orc

pytestmark = pytest.mark.gpu


def cpu_step(weights, x):
    return layer_oracle.cpu_step(L.SHAPES, weights, x)


@pytest.mark.parametrize("vocab_fraction", [1.0])
def test_layer_stack_greedy_token_matches_cpu(vocab_fraction):
    import torch
    weights = L.quantized_weights(vocab_fraction)
    x = gaussian(20, L.HIDDEN)
    b = nq.Backend(0)
    dev = L.upload(weights)
    xg = torch.from_numpy(x).cuda()
    token = L.run(b, dev, xg)
    logits = dev.buffers["logits"].cpu().numpy()
    b.close()
    ref = cpu_step(weights, x)
    want = orc.argmax(ref)
    top2 = np.sort(ref)[-2:]
    normwise = np.abs(logits - ref).max() / np.abs(ref).max()
    print(f"token gpu {token} cpu {want}; top-2 gap {top2[1] - top2[0]:.4g}; normwise {normwise:.2e}")
    assert normwise <= 2e-3
    assert token == want
