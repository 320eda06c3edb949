"""The two measuring kernels behind the ceilings the roofline figures are read against: the HBM
read stream (lava_hip_read_stream) and the MFMA loop (lava_hip_mfma_loop).

The read stream XORs every 32-bit word it reads into its thread's sink word, each word read by
exactly one thread, so the XOR of all sink words is the XOR of the buffer's words whatever the
launch shape.  The MFMA loop reads each lane's operands once and hashes its accumulators: two
launches on the same data give the same sink, and operand data that differ in one word give a
different one."""
from __future__ import annotations

import ctypes as C

import numpy as np
import pytest

from conftest import announce

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("nbytes,blocks,unroll", [(1 << 20, 4, 8), ((1 << 20) + 48, 3, 4), (4096, 64, 16)])
def test_read_stream_reads_every_word_once(gpu, rng, nbytes, blocks, unroll):
    lh = gpu
    announce(f"read_stream bytes={nbytes} blocks={blocks} unroll={unroll}")
    host = rng.integers(0, 2**32, size=nbytes // 4, dtype=np.uint32)
    src = lh.HIPDeviceArray.from_numpy(host, dtype="u32")
    sink = lh.HIPDeviceArray("u32", (blocks * 256,))
    lh._lib.call("lava_hip_read_stream", src.ptr, nbytes, sink.ptr, blocks, unroll, None)
    lh.synchronize()
    assert np.bitwise_xor.reduce(sink.to_numpy()) == np.bitwise_xor.reduce(host)


def test_read_stream_rejects_bad_arguments(gpu):
    lh = gpu
    src = lh.HIPDeviceArray("u8", (4096,))
    sink = lh.HIPDeviceArray("u32", (256,))
    for args in ((src.ptr, 4008, sink.ptr, 1, 8), (src.ptr, 4096, sink.ptr, 0, 8), (src.ptr, 4096, sink.ptr, 1, 5),
                 (src.ptr + 4, 4080, sink.ptr, 1, 8)):
        with pytest.raises(lh.InvalidArgument):
            lh._lib.call("lava_hip_read_stream", *args, None)


@pytest.mark.parametrize("form", range(6))
def test_mfma_loop_is_deterministic_and_sees_its_data(gpu, rng, form):
    lh = gpu
    announce(f"mfma_loop form={form}")
    words = 4096
    host = rng.integers(0, 2**16, size=2 * words, dtype=np.uint16)
    if form in (0, 3):   # fp16 in [1, 2)
        host = 0x3C00 | (host & 0x03FF)
    elif form in (1, 4):   # bf16 in [1, 2)
        host = 0x3F80 | (host & 0x007F)
    a = lh.HIPDeviceArray.from_numpy(host, dtype="bf16")
    b = lh.HIPDeviceArray.from_numpy(host[::-1].copy(), dtype="bf16")
    sinks = []
    for rep in range(3):
        if rep == 2:   # change the first word lane 0 reads
            h2 = host.copy()
            h2[0] ^= 0x0040   # a mantissa bit of a 16-bit value, bit 6 of an int8
            a.copy_from(h2)
        sink = lh.HIPDeviceArray("f32", (2 * 256 * 2,))
        lh._lib.call("lava_hip_mfma_loop", form, a.ptr, b.ptr, 4 * words, 2, 2, 3, sink.ptr, None)
        lh.synchronize()
        sinks.append(sink.to_numpy().view(np.uint32))
    assert np.array_equal(sinks[0], sinks[1])
    assert not np.array_equal(sinks[0], sinks[2])


def test_mfma_loop_rejects_bad_arguments(gpu):
    lh = gpu
    a = lh.HIPDeviceArray("u8", (4096,))
    sink = lh.HIPDeviceArray("f32", (1024,))
    for args in ((6, a.ptr, a.ptr, 4096, 1, 1, 1), (0, a.ptr, a.ptr, 4096, 1, 3, 1), (0, a.ptr, a.ptr, 4096, 1, 1, 0),
                 (0, a.ptr + 8, a.ptr, 4080, 1, 1, 1), (0, a.ptr, a.ptr, 0, 1, 1, 1), (0, a.ptr, a.ptr, 4096, 0, 1, 1)):
        with pytest.raises(lh.InvalidArgument):
            lh._lib.call("lava_hip_mfma_loop", *args, sink.ptr, None)
    with pytest.raises(lh.InvalidArgument):
        lh._lib.call("lava_hip_mfma_loop", 0, a.ptr, a.ptr, 4096, 1, 1, 1, C.c_void_p(None), None)
