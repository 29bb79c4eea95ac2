"""CPU checks of the SSD backward's host logic: the chunk table over the scan's
sequences (one row per 64-token chunk, rows of a sequence consecutive, each row
(sequence, first token, end token, 0, 1, index, first row, rows)) and the sequence
layout shared by the forward and the backward."""
import torch

from hmx.ops.ssd import seq_layout
from hmx.ops.ssd_train import _chunk_table


def test_chunk_table_tiles_every_sequence():
    bounds = [(0, 130), (130, 130), (130, 131), (300, 428)]
    rows, seqs = _chunk_table(bounds)
    assert rows == [(0, 0, 64, 0, 1, 0, 0, 3), (0, 64, 128, 0, 1, 1, 0, 3),
                    (0, 128, 130, 0, 1, 2, 0, 3),
                    (2, 130, 131, 0, 1, 0, 3, 1),
                    (3, 300, 364, 0, 1, 0, 4, 2), (3, 364, 428, 0, 1, 1, 4, 2)]
    assert seqs == [(0, 3), (3, 0), (3, 1), (4, 2)]
    # every token of every sequence in exactly one row
    covered = sorted(t for r in rows for t in range(r[1], r[2]))
    assert covered == [t for a, e in bounds for t in range(a, e)]


def test_seq_layout_rows_and_restarts():
    seq_idx = torch.tensor([[0, 0, 1, 1, 1], [4, 4, 4, 4, 4]])
    bounds, first, last, end_at = seq_layout(2, 5, seq_idx)
    assert bounds == [(0, 2), (2, 5), (5, 10)]
    assert first == [0, 2] and last == [1, 2]
    assert end_at == {(0, 2): 0, (0, 5): 1, (1, 5): 2}
    bounds, first, last, _ = seq_layout(3, 4)
    assert bounds == [(0, 4), (4, 8), (8, 12)] and first == [0, 1, 2] and last == [0, 1, 2]
