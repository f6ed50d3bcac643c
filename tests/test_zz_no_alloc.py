"""The allocation-free decode attention entry point
(jllm_hip_flash_attention_decode_noalloc: split-K partials in a fixed
per-device array) against the allocating one, through the C ABI: two calls
in a row, the second smaller, each bit-identical to
jllm_hip_flash_attention_decode on the same inputs (same kernels, same
split policy); oversize requests are refused before any device work."""
import numpy as np
import pytest
import torch

import jllm
import synth
from gpu_util import print_case, to_dev

pytestmark = pytest.mark.gpu


def _inputs(seed, ctx, H, KV, HD):
    g = synth.rng(seed)
    return (to_dev(synth.x_f16(g, H * HD)), to_dev(synth.kv_int8(g, ctx, KV, HD)),
            to_dev(synth.kv_int8(g, ctx, KV, HD)), to_dev(synth.kv_scales(g, ctx, KV)),
            to_dev(synth.kv_scales(g, ctx, KV)))


@pytest.mark.parametrize("first,second", [((32, 8, 128, 4096, 0), (32, 8, 128, 300, 0)),
                                          ((32, 8, 128, 8192, 512), (16, 4, 64, 40, 0)),
                                          # 64 heads x 128 key ranges: 32 partials per head after the
                                          # 4-wave grouping (1.06 MB) -- fits the 4 MiB array
                                          ((64, 8, 128, 8192, 0), (32, 8, 128, 640, 0))])
def test_noalloc_matches_allocating_entry(dev, first, second):
    for i, (H, KV, HD, ctx, window) in enumerate((first, second)):
        print_case("noalloc", i, H, KV, HD, ctx, window)
        q, k, v, ks, vs = _inputs(ctx + i, ctx, H, KV, HD)
        a = torch.full((H * HD,), 7, dtype=torch.int16, device=dev)
        b = torch.full((H * HD,), 9, dtype=torch.int16, device=dev)
        args = (q, k, v, H, KV, HD, HD, ctx, 1.0 / np.sqrt(HD), 1, ks, vs, window)
        jllm.call("jllm_hip_flash_attention_decode_noalloc", b, *args)
        jllm.call("jllm_hip_flash_attention_decode", a, *args)
        torch.cuda.synchronize()
        assert torch.equal(a, b), (i, ctx)


def test_noalloc_rejects_oversize(dev):
    # 256 heads (16 per KV head) x 128 key ranges grouped into 32 partials
    # of (2 + 128) floats = 4.26 MB > 4 MiB
    H, KV, HD, ctx = 256, 16, 128, 8192
    q, k, v, ks, vs = _inputs(1, 64, 8, 8, 128)
    out = torch.zeros(H * HD, dtype=torch.int16, device=dev)
    st = jllm.lib().jllm_hip_flash_attention_decode_noalloc(out.data_ptr(), q.data_ptr(), k.data_ptr(),
                                                            v.data_ptr(), H, KV, HD, HD, ctx, 0.1, 1,
                                                            ks.data_ptr(), vs.data_ptr(), 0, None)
    assert st == -1
