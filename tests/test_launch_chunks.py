"""Chunk heights of small launches on the code-sorted layout: the launch-level rule that
PackedProjections applies to q, k and v (about 0.75 x CUs chunks over their total rows, at
most 64 rows, one workgroup per chunk), and the slice rule of batch-1 launches, checked on the
host with a stand-in CU count."""
import torch

from compressai_amd import kernels as K


def test_launch_rows_per_chunk(monkeypatch):
    monkeypatch.setitem(K._CU_COUNT, 0, 256)
    dev = torch.device("cuda", 0)
    assert K.sorted_launch_rows_per_chunk([2048, 512, 512], 256, dev) == 16    # q, k, v: 192 chunks
    assert K.sorted_launch_rows_per_chunk([2048], 256, dev) == 11              # o: 187 chunks
    assert K.sorted_launch_rows_per_chunk([6144, 6144], 256, dev) is None      # gate + up: the defaults
    assert K.sorted_launch_rows_per_chunk([2048], 768, dev) is None            # 1.5 M codes
    assert K.sorted_launch_rows_per_chunk([100], 256, dev) == 1
    assert K.sorted_launch_rows_per_chunk([1024], 2048, dev) is None           # 2 M codes
    assert K.sorted_launch_rows_per_chunk([64], 4096, dev) == 1                # 16-bit positions: 15 rows at most
    monkeypatch.setitem(K._CU_COUNT, 0, 32)
    assert K.sorted_launch_rows_per_chunk([2048, 512, 512], 256, dev) == 64    # few CUs: the 64-row cap


def test_sorted_slices_rule(monkeypatch):
    """Workgroups per chunk of a batch-1 sorted launch: one where fewer than three fit on the
    CUs (the small launches above), else as many as fit, each wave keeping an iteration."""
    from types import SimpleNamespace as P

    monkeypatch.setitem(K._CU_COUNT, 0, 256)
    dev = torch.device("cuda", 0)
    assert K.sorted_slices([P(n_chunks=187, iters_per_chunk=19)], dev) == 1       # o: 11-row chunks
    assert K.sorted_slices([P(n_chunks=128, iters_per_chunk=41)], dev) == 1       # 2 would fit
    assert K.sorted_slices([P(n_chunks=86, iters_per_chunk=42)], dev) == 1
    assert K.sorted_slices([P(n_chunks=25, iters_per_chunk=494)] * 2, dev) == 5   # gate + up
    assert K.sorted_slices([P(n_chunks=33, iters_per_chunk=200)], dev) == 7       # down
    assert K.sorted_slices([P(n_chunks=32, iters_per_chunk=50)], dev) == 2        # few iterations per wave
    assert K.sorted_slices([P(n_chunks=512, iters_per_chunk=300)], dev) == 1      # LM head


def test_sorted_batch_fits_rule():
    """The batch kernel's LDS rule as the runtime reads it: 4-row workgroups above 80 KiB run as
    2-row launches, which must fit in 150 KiB."""
    from types import SimpleNamespace as P

    assert K.sorted_batch_fits([P(n=2048, rows_per_chunk=246)] * 2, 4)        # gate + up: 79.6 KiB at 4 rows
    assert K.sorted_batch_fits([P(n=2048, rows_per_chunk=297)], 4)            # LM head: split, 46 KiB at 2 rows
    assert K.sorted_batch_fits([P(n=6144, rows_per_chunk=63)], 4)             # down
    assert K.sorted_batch_fits([P(n=32768, rows_per_chunk=31)], 4)            # split: 139 KiB at 2 rows
    assert not K.sorted_batch_fits([P(n=65536, rows_per_chunk=7)], 4)         # 2 rows: 256 KiB
    assert not K.sorted_batch_fits([P(n=65536, rows_per_chunk=7)], 2)
