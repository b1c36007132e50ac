"""What FlashInfer's approximate reciprocals can change in the NVFP4 activation
quantizer, bounded on the NVFP4 configuration's activations (CPU sample).

The oracle and the HIP quantizer use correctly rounded reciprocals where
FlashInfer uses the hardware's approximate one (one ulp at most); this pins how
many blocks depend on that choice.  tests/nvfp4_reciprocals.py describes the
analysis; test_gpu_nvfp4.py repeats it on every block of the 32760 x 5120
activation matrix.
"""

import numpy as np
import torch

from oracle import nvfp4 as NV
from tests.nvfp4_reciprocals import divergence


def test_reciprocal_choice_bound_on_a_sample_of_the_configuration():
    # The configuration's activation recipe (N(0, 1), seed 0) on 1024 rows, with
    # the calibrated global scale 2688 / amax.
    x = torch.randn((1024, 5120), generator=torch.Generator().manual_seed(0)).to(torch.bfloat16)
    gsf = np.float32(2688.0 / float(x.float().abs().max()))
    blocks, sf_moved, moved, ref_sf, ref_q = divergence(x, gsf)
    # The correctly rounded combination is the oracle's quantizer, bit for bit.
    packed, tiled = NV.quantize_activation(x.float().numpy(), gsf)
    assert np.array_equal(NV.unswizzle_128x4(tiled)[:1024], ref_sf.numpy().astype(np.uint8))
    q = ref_q.reshape(1024, -1).numpy()
    assert np.array_equal((q[:, 0::2] | (q[:, 1::2] << 4)).astype(np.uint8), packed)
    # Blocks whose E4M3 scale (through 1/6) or E2M1 codes (at E2M1 ties, through
    # 1/gsf and the block reciprocal) depend on the reciprocals' last ulp.
    assert blocks == 327680
    assert sf_moved == 2265  # 0.69 %
    assert moved == 20767  # 6.34 %
