"""The scorer's measurement kernels (lap_floor_stream, lap_floor_empty) read
what they claim to: the XOR of every word a workgroup reads, against numpy
over the same table and code rows (a dropped stage, a wrong row stride or a
short table copy changes the word)."""
import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu

CHUNK = 4096  # tokens per workgroup: 1024 threads x 4 stages


def _expected(table_u32, codes_u32, R, T):
    """Per workgroup i (row i % R, chunk i // R): the table row's words, and
    the code rows t0 + j * 1024 + tid (j < 4, tid < 1024) clamped to t1 - 1,
    each XOR-ed once per read (so the clamped last row counts 4096 - n + 1
    times)."""
    nchunk = (T + CHUNK - 1) // CHUNK
    out = np.zeros(R * nchunk, dtype=np.uint32)
    for i in range(R * nchunk):
        r, ch = i % R, i // R
        t0, t1 = ch * CHUNK, min(T, ch * CHUNK + CHUNK)
        x = np.bitwise_xor.reduce(table_u32[r].ravel())
        if t1 - 1 > t0:
            x ^= np.bitwise_xor.reduce(codes_u32[r, t0:t1 - 1].ravel())
        if (CHUNK - (t1 - t0) + 1) % 2:
            x ^= np.bitwise_xor.reduce(codes_u32[r, t1 - 1])
        out[i] = x
    return out


@pytest.mark.parametrize("ahead", [1, 4])
@pytest.mark.parametrize("R,T,tcap", [(3, 5000, 5120), (8, 8192, 8192), (2, 100, 128)])
def test_floor_stream_reads_every_word(dev, ahead, R, T, tcap):
    from laprune_amd import _native as N
    g = torch.Generator().manual_seed(R * 7919 + T + ahead)
    table = torch.randint(-2**15, 2**15, (R, 32768), generator=g, dtype=torch.int16)
    codes = torch.randint(0, 256, (R, tcap, 32), generator=g, dtype=torch.uint8)
    nchunk = (T + CHUNK - 1) // CHUNK
    t_d, c_d = table.to(dev), codes.to(dev)
    out = torch.zeros(R * nchunk, dtype=torch.int32, device=dev)
    print(f"lap_floor_stream R={R} T={T} tcap={tcap} ahead={ahead}", flush=True)
    N.call("lap_floor_stream", N.ptr(t_d), N.ptr(c_d), c_d.stride(0), c_d.stride(1), R, T,
           ahead, N.ptr(out), N.stream_of(c_d))
    torch.cuda.synchronize()
    want = _expected(table.numpy().view(np.uint32).reshape(R, -1),
                     codes.numpy().view(np.uint32).reshape(R, tcap, 8), R, T)
    got = out.cpu().numpy().view(np.uint32)
    assert np.array_equal(got, want)


def test_floor_empty_runs(dev):
    from laprune_amd import _native as N
    print("lap_floor_empty R=8 T=131072", flush=True)
    N.call("lap_floor_empty", 8, 131072, N.stream_of(torch.empty(1, device=dev)))
    torch.cuda.synchronize()
