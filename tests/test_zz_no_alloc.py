"""ku_hip_linear_e4m3_noalloc: the e4m3 linear with its scratch in a static device array.

Checked through the C ABI against the allocating entry point (ku_hip_linear_e4m3), bit for bit,
on two calls in a row, the second with a smaller input (the static scratch keeps the first
call's contents); sizes past the static scratch are rejected with an error."""
import numpy as np
import pytest

import kurumi_amd as K
from hipmem import DevBuf, synchronize
from kurumi_amd import DType
from kutest import f32_to_bf16_bits
from test_gpu_linear_e4m3 import quantise_rows

pytestmark = pytest.mark.gpu


def case(seed, m, n, k, scale):
    rng = np.random.default_rng(seed)
    w = (rng.standard_normal((n, k), dtype=np.float32) * 0.02).astype(np.float32)
    xbits = f32_to_bf16_bits(rng.standard_normal((m, k), dtype=np.float32) * scale)
    wq, sw = quantise_rows(w)
    return DevBuf.from_numpy(xbits), DevBuf.from_numpy(wq), DevBuf.from_numpy(sw)


def test_noalloc_matches_allocating_entry_point_on_two_calls(hip):
    print("linear_e4m3_noalloc: two calls, the second smaller", flush=True)
    # the second call is smaller and its activations much smaller in magnitude: a stale sx or
    # stale partials from the first call would change every output
    for seed, m, n, k, scale in ((1, 2048, 11008, 4096, 4.0), (2, 300, 520, 384, 0.25)):
        x, wq, sw = case(seed, m, n, k, scale)
        y_ref = DevBuf(m * n * 2)
        y_na = DevBuf(m * n * 2)
        hip.linear_e4m3(x.ptr, DType.BF16, wq.ptr, sw.ptr, y_ref.ptr, DType.BF16, m, n, k)
        synchronize()
        K.linear_e4m3_noalloc(x.ptr, DType.BF16, wq.ptr, sw.ptr, y_na.ptr, DType.BF16, m, n, k)
        synchronize()
        want = y_ref.numpy(np.uint16, (m, n))
        got = y_na.numpy(np.uint16, (m, n))
        np.testing.assert_array_equal(got, want, err_msg=f"call {seed} ({m}x{n}x{k})")


def test_noalloc_rejects_sizes_past_its_scratch():
    d = DevBuf(4096)
    with pytest.raises(K.KuError, match="static scratch"):
        K.linear_e4m3_noalloc(d.ptr, DType.BF16, d.ptr, d.ptr, d.ptr, DType.BF16, 4097, 128, 4096)
