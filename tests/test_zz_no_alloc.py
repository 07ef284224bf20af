"""The no-allocation decode attention (aegkv_paged_decode_attention_noalloc):
called through the C ABI, its output equals aegkv_paged_decode_attention's
with a caller workspace bit for bit, on two calls in a row (the second with a
smaller batch, so stale scratch contents from the first are present), and a
call that needs more than the library's scratch is refused before anything is
enqueued.  The entry point has no counterpart in the reference; the existing
entry point it mirrors is itself checked against the float64 oracle."""
import math

import numpy as np
import pytest
import torch

from aegaeon_amd import _lib
from oracle import kv_oracle as ko
from tests.kvtest_utils import random_bits, to_bits, to_device_bits

pytestmark = pytest.mark.gpu

SCRATCH_BYTES = 32 << 20


def _case(device, rng, lens, Hq, Hkv, D):
    lens = np.asarray(lens, dtype=np.int64)
    need = [-(-int(x) // 16) for x in lens]
    N = 2 * sum(need) + 5
    ids = rng.permutation(N)[:sum(need)]
    tables, o = [], 0
    for c in need:
        tables.append([int(x) for x in ids[o:o + c]])
        o += c
    padded = ko.pad_block_tables(tables)
    kc = to_device_bits(random_bits(rng, (N, 16, Hkv, D), "bf16"), "bf16", device)
    vc = to_device_bits(random_bits(rng, (N, 16, Hkv, D), "bf16"), "bf16", device)
    q = to_device_bits(random_bits(rng, (len(lens), Hq, D), "bf16"), "bf16", device)
    bt = torch.from_numpy(padded).to(device)
    sl = torch.from_numpy(lens.astype(np.int32)).to(device)
    return q, kc, vc, bt, sl, int(lens.max()), N


def _call(lib, name, out, q, kc, vc, bt, sl, max_len, N, ws=None):
    B, Hq, D = q.shape
    Hkv = kc.size(2)
    stream = torch.cuda.current_stream().cuda_stream
    common = (out.data_ptr(), out.stride(0), q.data_ptr(), q.stride(0), kc.data_ptr(),
              vc.data_ptr(), kc.stride(0), N, bt.data_ptr(), bt.size(1), sl.data_ptr(), B,
              max_len, Hq, Hkv, D, 16, 1.0 / math.sqrt(D), _lib.AEGKV_DTYPE_BF16, 0)
    if ws is None:
        return getattr(lib, name)(*common, stream)
    return getattr(lib, name)(*common, ws.data_ptr(), ws.numel(), stream)


@pytest.mark.parametrize("Hq,Hkv,D", [(28, 4, 128), (32, 4, 128), (8, 8, 64)])
def test_noalloc_matches_workspace_entry(device, Hq, Hkv, D):
    lib = _lib.load()
    rng = np.random.default_rng(Hq + D)
    batches = [rng.integers(1, 3000, 96).tolist() + [0, 1, 16, 17],   # first call
               rng.integers(1, 400, 9).tolist()]                       # smaller second call
    for lens in batches:
        q, kc, vc, bt, sl, ml, N = _case(device, rng, lens, Hq, Hkv, D)
        need = lib.aegkv_paged_decode_attention_workspace_size(len(lens), Hq, Hkv, D, ml,
                                                               _lib.AEGKV_DTYPE_BF16, 0)
        assert 0 < need <= SCRATCH_BYTES
        ws = torch.empty(need, dtype=torch.uint8, device=device)
        ref = torch.empty_like(q)
        got = torch.full_like(q, float("nan"))
        assert _call(lib, "aegkv_paged_decode_attention", ref, q, kc, vc, bt, sl, ml, N, ws) == 0
        assert _call(lib, "aegkv_paged_decode_attention_noalloc", got, q, kc, vc, bt, sl, ml,
                     N) == 0
        torch.cuda.synchronize()
        assert np.array_equal(to_bits(got), to_bits(ref)), lens[:4]


def test_noalloc_refuses_oversize_before_launch(device):
    """Llama-2-13B heads (40/40, D 128) at 2048 sequences need 41 MiB of
    workspace: refused with AEGKV_ERR_SCRATCH, the output untouched."""
    lib = _lib.load()
    B, H, D = 2048, 40, 128
    need = lib.aegkv_paged_decode_attention_workspace_size(B, H, H, D, 16, 0, 0)
    assert need > SCRATCH_BYTES
    q = torch.zeros((B, H, D), dtype=torch.bfloat16, device=device)
    out = torch.full_like(q, 3.0)
    kc = torch.zeros((4, 16, H, D), dtype=torch.bfloat16, device=device)
    bt = torch.zeros((B, 1), dtype=torch.int32, device=device)
    sl = torch.ones(B, dtype=torch.int32, device=device)
    rc = _call(lib, "aegkv_paged_decode_attention_noalloc", out, q, kc, kc, bt, sl, 16, 4)
    assert rc == -11 and "32 MiB" in _lib.strerror(rc)
    torch.cuda.synchronize()
    assert bool((out == 3.0).all())
