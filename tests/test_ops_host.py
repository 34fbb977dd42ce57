"""Host-side layout helpers of the decode GEMMs (CPU): the fragment order of
PackedWeight and the gate / up row interleave that the fused gate|up + SwiGLU
launch reads."""
import pytest

torch = pytest.importorskip("torch")


def test_packed_weight_layout_and_round_trip():
    from tinytron_amd import ops

    N, K = 32, 64
    w = torch.arange(N * K, dtype=torch.float32).reshape(N, K)
    pw = ops.PackedWeight(w)
    flat = pw.data.reshape(-1)
    # element W[n][k] sits at ((n/16)(K/32) + k/32) * 512 + ((k%32)/8) * 128 + (n%16) * 8 + k%8
    for n, k in [(0, 0), (5, 9), (17, 40), (31, 63), (16, 32)]:
        idx = ((n // 16) * (K // 32) + k // 32) * 512 + ((k % 32) // 8) * 128 + (n % 16) * 8 + k % 8
        assert flat[idx] == w[n, k]
    assert torch.equal(pw.unpack(), w)


def test_interleave_gate_up_rows():
    from tinytron_amd import ops

    inter, K = 24, 4
    gate = torch.arange(inter, dtype=torch.float32)[:, None].expand(inter, K) + 1000
    up = torch.arange(inter, dtype=torch.float32)[:, None].expand(inter, K) + 2000
    w = ops.interleave_gate_up(gate, up)
    assert w.shape == (2 * inter, K)
    for row in range(2 * inter):
        j, i = divmod(row, 16)
        expect = (1000 + 8 * j + i) if i < 8 else (2000 + 8 * j + i - 8)
        assert torch.all(w[row] == expect), row
    with pytest.raises(ValueError):
        ops.interleave_gate_up(gate[:12], up[:12])  # I % 8 != 0
