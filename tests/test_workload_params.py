"""CPU checks of the parameter construction that the full-size GPU parity tests use to realise the workloads' gate
distributions through the converted core's own parameters (no GPU needed)."""
import math

import torch

from oracle import layer as olayer
from test_gpu_workloads import spectrum_core, spectrum_inputs


def test_spectrum_gates_realise_the_workload():
    """The parameter construction above gives g = -ln2/life on the decaying heads, 0 on the archival head, beta =
    sigmoid(z_beta) (0 on the sinks) and gamma logits = z_gamma (checked on the oracle's mem_inputs, CPU)."""
    m = spectrum_core(16, 4, 256, 2048, 4, (2048.0, 45255.0, 1e6, None))
    x, q, k, v, qr, kr = spectrum_inputs(1, 40, 16, 4, 256, 0, torch.float32)
    pos = torch.arange(40)
    qm, km, g, beta = olayer.mem_inputs(m, x, q, k, pos)
    want = torch.tensor([-math.log(2) / 2048, -math.log(2) / 45255, -math.log(2) / 1e6, 0.0])
    assert torch.allclose(g[0], want.expand(40, 4), rtol=1e-5, atol=0)
    assert torch.allclose(beta[0, 4:], torch.sigmoid(x[0, 4:, :4]), atol=1e-7) and (beta[0, :4] == 0).all()
    assert torch.allclose(olayer.mix_logits(m, x), x[..., 4:], atol=1e-7)
    assert torch.allclose(qm, q * 256 ** -0.5, atol=1e-6) and torch.allclose(km, k, atol=1e-6)
