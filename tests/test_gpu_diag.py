"""GPU checks of the measurement kernels (libllmik_diag.so, csrc_diag/diag.hip) that bench.py
--floors times: the plain read must read every byte once (the xor of the
per-wave values equals the xor of every 32-bit word, computed on the CPU),
at sizes that end inside a 4 KiB unit and at grids with more waves than
units; the empty kernel must launch."""
from __future__ import annotations

import ctypes

import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu


def _lib():
    from llmik_cuda._lib import diag_check, diag_lib
    return diag_lib(), diag_check


def _stream():
    return ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)


@pytest.mark.parametrize("L", [4, 8, 16])
@pytest.mark.parametrize("nbytes,nwg", [(16, 1), (4096, 2), (16000, 3), (40000, 1), (8_667_136, 256),
                                        (30_314_496, 1024), (1 << 20, 2048)])
def test_read_xor_covers_every_word(cuda, nbytes, nwg, L):
    lib, check = _lib()
    gen = torch.Generator(device=cuda).manual_seed(nbytes + nwg)
    buf = torch.randint(-2 ** 31, 2 ** 31 - 1, (nbytes // 4 + 64,), generator=gen, device=cuda,
                        dtype=torch.int32)   # 256 bytes past the range: must not be read
    sink = torch.full((nwg * 8,), -1, dtype=torch.int32, device=cuda)
    check(lib.llmik_diag_read(ctypes.c_void_p(buf.data_ptr()), nbytes,
                              ctypes.c_void_p(sink.data_ptr()), nwg, L, _stream()))
    torch.cuda.synchronize()
    words = buf.cpu().numpy().view(np.uint32)[:nbytes // 4]
    want = np.bitwise_xor.reduce(words) if words.size else np.uint32(0)
    got = np.bitwise_xor.reduce(sink.cpu().numpy().view(np.uint32))
    assert got == want


def test_read_rejects_bad_arguments(cuda):
    lib, _ = _lib()
    buf = torch.zeros(1024, dtype=torch.int32, device=cuda)
    sink = torch.zeros(8, dtype=torch.int32, device=cuda)
    p, s = ctypes.c_void_p(buf.data_ptr()), ctypes.c_void_p(sink.data_ptr())
    assert lib.llmik_diag_read(p, 100, s, 1, 4, _stream()) != 0          # not a multiple of 16
    assert lib.llmik_diag_read(ctypes.c_void_p(buf.data_ptr() + 4), 64, s, 1, 4, _stream()) != 0
    assert lib.llmik_diag_read(p, 64, s, 0, 4, _stream()) != 0
    assert lib.llmik_diag_read(p, 64, s, 1, 5, _stream()) != 0
    assert lib.llmik_diag_empty(0, _stream()) != 0


def test_empty_kernel_launches(cuda):
    lib, check = _lib()
    for nwg in (1, 256, 1024):
        check(lib.llmik_diag_empty(nwg, _stream()))
    torch.cuda.synchronize()


@pytest.mark.parametrize("W", [4, 8, 16])
@pytest.mark.parametrize("L", [4, 8])
@pytest.mark.parametrize("nbytes,nwg", [(16, 1), (16000, 3), (1 << 20, 256), (4_194_304 + 4096, 2048)])
def test_read_write_copies_the_leading_bytes(cuda, nbytes, nwg, L, W):
    """llmik_diag_read_write writes the first W bytes of every 16-byte chunk
    of src, in order, and nothing past bytes / 16 * W (a guard tail stays)."""
    lib, check = _lib()
    gen = torch.Generator(device=cuda).manual_seed(nbytes + W)
    src = torch.randint(0, 256, (nbytes,), generator=gen, device=cuda, dtype=torch.uint8)
    out_len = nbytes // 16 * W
    dst = torch.full((out_len + 256,), 0xA5, dtype=torch.uint8, device=cuda)
    check(lib.llmik_diag_read_write(ctypes.c_void_p(src.data_ptr()), nbytes, ctypes.c_void_p(dst.data_ptr()),
                                    W, nwg, L, _stream()))
    torch.cuda.synchronize()
    want = src.cpu().numpy().reshape(-1, 16)[:, :W].reshape(-1)
    got = dst.cpu().numpy()
    assert np.array_equal(got[:out_len], want)
    assert (got[out_len:] == 0xA5).all()


def test_read_write_rejects_bad_arguments(cuda):
    lib, _ = _lib()
    buf = torch.zeros(1024, dtype=torch.int32, device=cuda)
    p = ctypes.c_void_p(buf.data_ptr())
    assert lib.llmik_diag_read_write(p, 100, p, 8, 1, 4, _stream()) != 0      # not a multiple of 16
    assert lib.llmik_diag_read_write(p, 64, p, 5, 1, 4, _stream()) != 0       # write width
    assert lib.llmik_diag_read_write(p, 64, p, 8, 1, 16, _stream()) != 0      # depth
    assert lib.llmik_diag_read_write(p, 64, p, 8, 0, 4, _stream()) != 0
