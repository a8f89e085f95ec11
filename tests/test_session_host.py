"""Host-side pieces of TensorSession that need no GPU: AttentionDims and the
error variants the session raises (session/mod.rs:60-99, error.rs:31-38,
:143-152, cast.rs:31-37)."""
from __future__ import annotations

import pytest

from barracuda_amd import AttentionDims, CastOverflow, InvalidShape, TensorSession
from barracuda_amd import session as S


def test_attention_dims():
    d = AttentionDims(batch_size=4, n_heads=32, seq_len=2048, head_dim=128)
    assert d.total_elements() == 4 * 32 * 2048 * 128
    assert d.as_u32() == (4, 2048, 32, 128)  # (batch, seq, heads, dim) order
    with pytest.raises(CastOverflow, match=r"Cast overflow: usize → u32 \(4294967296\)"):
        AttentionDims(1, 1, 2**32, 1).as_u32()
    assert AttentionDims(1, 1, 2**32 - 1, 1).as_u32()[1] == 2**32 - 1


def test_error_text():
    e = InvalidShape([1, 2, 3], [1, 2])
    assert str(e) == "Invalid shape: expected [1, 2, 3], got [1, 2]"
    assert e.expected == [1, 2, 3] and e.actual == [1, 2]


def test_session_surface():
    for name in ("new", "with_device", "reset", "num_ops", "tensor", "tensor_with_shape", "import",
                 "matmul", "softmax", "attention", "run"):
        assert callable(getattr(TensorSession, name)), name
    for name in ("shape", "len", "is_empty", "to_vec", "to_tensor"):
        assert callable(getattr(S.SessionTensor, name)), name
