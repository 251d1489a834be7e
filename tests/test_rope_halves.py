"""fdl.ops.tables_repeat_halves, the check behind FDL_QKV_ROPE_HALVES_EQUAL, on CPU tensors:
the reference's tables (cat(freqs, freqs)) repeat their halves, other tables do not, and a
remembered answer is dropped when a table is modified in place or replaced."""
import torch

from fdl import ops
from fdl.generate import get_rotary_embedding


def test_reference_tables_repeat_their_halves():
    sin, cos = get_rotary_embedding(384, 128, 500000.0, "cpu")
    assert ops.tables_repeat_halves(sin, cos)
    assert ops.tables_repeat_halves(sin, cos)  # remembered


def test_modified_or_other_tables_do_not():
    sin, cos = get_rotary_embedding(64, 128, 10000.0, "cpu")
    sin, cos = sin.clone(), cos.clone()
    assert ops.tables_repeat_halves(sin, cos)
    sin[5, 100] += 1.0  # in place: the version counter changes, the answer is recomputed
    assert not ops.tables_repeat_halves(sin, cos)
    gen = torch.Generator().manual_seed(3)
    s2, c2 = torch.rand((64, 128), generator=gen), torch.rand((64, 128), generator=gen)
    assert not ops.tables_repeat_halves(s2, c2)
    # one table repeating, the other not
    assert not ops.tables_repeat_halves(cos, s2)
