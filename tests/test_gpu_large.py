"""A batch past 32-bit element offsets (MI355X: 288 GB of HBM per GPU).

At B = 32800 the row offsets of x, y, the coefficient planes and the slot
buffer F all pass 2^31 elements (x from row 32768 on, F from row 29077 on),
so any 32-bit index arithmetic in a kernel would land in the wrong rows.
The rows at both ends must equal their batch-1 results bit for bit, and
round-trip at >= 125 dB. About 90 GB of device memory; the test is skipped
on a card with less free memory and releases everything it allocated."""
import gc

import numpy as np
import pytest
import torch

from oracle.cqt_oracle import snr_db

pytestmark = pytest.mark.gpu

N = 65536
B = 32800
NEED = 100 * 2**30


def test_batch_past_32bit_offsets():
    from flash_cqt import OctCQT
    from flash_cqt import tables as T
    from flash_cqt.fused import FusedOctCQT
    dev = torch.device("cuda:0")
    free, _ = torch.cuda.mem_get_info(dev)
    if free < NEED:
        pytest.skip(f"needs {NEED / 2**30:.0f} GiB free, {free / 2**30:.0f} GiB available")
    assert (B - 1) * N >= 2**31 and (B - 1) * T.FROW >= 2**31
    f = FusedOctCQT(OctCQT([3, 4, 2], [8, 16, 32], fs=44100, audio_len=N, device=dev), dev)
    assert (B - 1) * f.ncoef >= 2**31
    try:
        g = torch.Generator(device=dev)
        g.manual_seed(5)
        x = torch.randn(B, N, device=dev, generator=g)
        print(f"B={B}: analysis", flush=True)
        KR, KI = f.fwd(x)
        print(f"B={B}: synthesis", flush=True)
        y = f.bwd(KR, KI)
        rows = (0, 1, 29077, 32767, 32768, B - 1)
        kr = KR[list(rows)].clone()
        ki = KI[list(rows)].clone()
        yr = y[list(rows)].clone()
        xr = x[list(rows)].clone()
        del KR, KI, y, x
        f.release_workspace()
        gc.collect()
        torch.cuda.empty_cache()
        for j, r in enumerate(rows):
            k1, i1 = f.fwd(xr[j:j + 1].contiguous())
            assert torch.equal(k1[0], kr[j]) and torch.equal(i1[0], ki[j]), r
            assert torch.equal(f.bwd(k1, i1)[0], yr[j]), r
            db = snr_db(xr[j].double().cpu().numpy(), yr[j].double().cpu().numpy())
            assert db >= 125, (r, db)
        torch.cuda.synchronize()
    finally:
        f.release_workspace()
        del f
        gc.collect()
        torch.cuda.empty_cache()
