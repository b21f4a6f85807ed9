"""GPU: the read-only streaming kernel behind bench.py's ``read_ceiling_gbs``
reads every 16-byte word once: the XOR of the words it returns equals the
XOR of the whole buffer, for a size with a partial last iteration."""
import numpy as np
import pytest
import torch

import gfx906_fa
from gpu_common import announce, need_gpu

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("words", [4, 1 << 20, (1 << 22) + 12])
def test_stream_read_reads_every_word(words):
    need_gpu()
    announce(f"stream_read {words} x 16 B")
    rng = np.random.default_rng(words)
    host = rng.integers(-2**31, 2**31, size=words * 4, dtype=np.int64).astype(np.int32)
    src = torch.from_numpy(host).cuda()
    out = gfx906_fa.stream_read(src)
    torch.cuda.synchronize()
    got = np.bitwise_xor.reduce(out.cpu().numpy().view(np.uint32))
    want = np.bitwise_xor.reduce(host.view(np.uint32))
    assert got == want
