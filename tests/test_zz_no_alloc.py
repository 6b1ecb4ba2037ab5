"""kvrt_attend_tensors_noalloc_async (the entry point that allocates nothing)
against kvrt_attend_tensors_async, both called through the C ABI: three calls
in a row on one GPU's shared scratch, each smaller than the one before, every
output equal to the allocating entry point's (bit for bit where both use the
same split count; within the attention tolerance of 1e-2 and of the oracle
where the scratch forced fewer splits), and a call too large for the scratch
refused with nothing written."""
from __future__ import annotations

import ctypes
import math

import numpy as np
import pytest
import torch

from oracle import kv_oracle as O
from tests.helpers import bits, randn_bf16, to_np

pytestmark = pytest.mark.gpu
ATOL = 1e-2


def _call(fn, q, k, v, lengths, out, scale, window, prefix=None):
    from kvrt.runtime import current_stream_handle, tensor_desc

    qd, kd, vd, od = tensor_desc(q), tensor_desc(k), tensor_desc(v), tensor_desc(out)
    pd = None if prefix is None else ctypes.byref(tensor_desc(prefix))
    return fn(ctypes.byref(qd), ctypes.byref(kd), ctypes.byref(vd), ctypes.c_void_p(lengths.data_ptr()), pd,
              ctypes.byref(od), ctypes.c_float(scale), ctypes.c_int32(window),
              ctypes.c_void_p(current_stream_handle(q.device)))


def _case(gen, n, hq, hkv, qn, d, lmax, lens, prefix_len=0):
    k = randn_bf16(gen, (n, hkv, lmax, d)).cuda()
    v = randn_bf16(gen, (n, hkv, lmax, d)).cuda()
    q = randn_bf16(gen, (n, hq, qn, d), 1.0 / math.sqrt(d)).cuda()
    lengths = torch.tensor(lens, dtype=torch.int32, device="cuda")
    prefix = None
    if prefix_len:
        prefix = torch.randint(0, 2, (n, prefix_len), generator=gen).to(torch.int64)
        prefix[:, 0] = 1
        prefix = prefix.cuda()
    return q, k, v, lengths, prefix


def _oracle(q, k, v, lens, scale, window, prefix):
    outs = []
    for b, L in enumerate(lens):
        qn = q.shape[2]
        pm = None if prefix is None else prefix[b].cpu().numpy()
        outs.append(O.attend(to_np(q[b]), to_np(k[b, :, :L]), to_np(v[b, :, :L]), np.arange(L - qn, L), scale,
                             window, prefix_attention=pm))
    return np.stack(outs)


def test_noalloc_entry_point_matches_the_allocating_one_over_successive_calls():
    from kvrt import _lib as L

    lib = L.load()
    gen = torch.Generator().manual_seed(2024)
    cases = [
        # (n, Hq, Hkv, Q, D, Lmax, lengths, window, prefix P): the first needs
        # fewer splits to fit the 16 MiB scratch (D 512, 16 rows, 4000 keys)
        (4, 8, 1, 2, 512, 4000, [4000, 3100, 2500, 3999], 0, 34),
        (4, 16, 8, 2, 128, 900, [900, 640, 77, 512], 0, 0),        # talker-shaped
        (2, 8, 1, 1, 256, 300, [300, 129], 128, 120),               # thinker sliding, masked
        (4, 16, 8, 1, 128, 2304, [2304, 2100, 1500, 2201], 0, 0),  # talker, MFMA decode's DMA ring
    ]
    scale = 1.0
    for i, (n, hq, hkv, qn, d, lmax, lens, window, plen) in enumerate(cases):
        print(f"[noalloc] call {i}: n {n} Hq {hq} Hkv {hkv} Q {qn} D {d} Lmax {lmax} window {window} P {plen}",
              flush=True)
        q, k, v, lengths, prefix = _case(gen, n, hq, hkv, qn, d, lmax, lens, plen)
        want = torch.empty_like(q)
        got = torch.full_like(q, float("nan"))
        assert _call(lib.kvrt_attend_tensors_async, q, k, v, lengths, want, scale, window, prefix) == 0
        assert _call(lib.kvrt_attend_tensors_noalloc_async, q, k, v, lengths, got, scale, window, prefix) == 0
        torch.cuda.synchronize()
        ref = _oracle(q, k, v, lens, scale, window, prefix)
        assert float(np.abs(to_np(got) - ref).max()) <= ATOL
        assert float(np.abs(to_np(want) - ref).max()) <= ATOL
        if i == 0:
            assert float((got.float() - want.float()).abs().max()) <= ATOL
        else:  # same split count as the allocating call: the same bits
            np.testing.assert_array_equal(bits(got), bits(want))


def test_noalloc_entry_point_refuses_calls_beyond_its_scratch():
    from kvrt import _lib as L

    lib = L.load()
    gen = torch.Generator().manual_seed(7)
    # 64 items x 16 kv heads x 16 rows x D 512: one workgroup per (item, kv
    # head) already needs 4 x 16 x 512 x 4 B x 1024 = 128 MiB of partials
    n, hkv = 64, 16
    q = randn_bf16(gen, (n, 8 * hkv, 2, 512)).cuda()
    k = torch.zeros((n, hkv, 4, 512), dtype=torch.bfloat16, device="cuda")
    lengths = torch.full((n,), 4, dtype=torch.int32, device="cuda")
    out = torch.full_like(q, 7.0)
    assert _call(lib.kvrt_attend_tensors_noalloc_async, q, k, k, lengths, out, 1.0, 0) == L.KVRT_EINVAL
    torch.cuda.synchronize()
    assert bool((out == 7.0).all())
