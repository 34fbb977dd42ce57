"""GPU parity at the head dims and group sizes of the reference's model presets
beyond 64 / 128 and powers of two (tinytron/model/config.py head_dim =
hidden_size / num_attention_heads; scripts/debug/inference.sh:52-107 and the
pretrain presets: 0.25B / 1B / 7B D 32, 0.1B D 48, D 24 at d 768 / 32 heads,
13B G = 5).

* head_dim a multiple of 8 (bf16 cache) / 16 (fp8 cache), <= 128: the MFMA
  kernels on 32 / 64 / 128-wide tiles with rows of the real head_dim (32
  exact; 24, 48, 80, 96, 112 padded) -- decode attention, the fused decode step
  and prefill attention;
* other even head dims (and fp32 caches): the VALU decode kernel.

Decode and prefill against the fp64 oracle within |err| <= 2e-3 + 2e-2 |ref|;
the fused step against the two-launch path bit for bit (which is itself pinned
to the oracle here and in test_gpu_rope_append.py's head_dim sweep).
"""
import numpy as np
import pytest

torch = pytest.importorskip("torch")

from tests.test_gpu_decode_attention import assert_close, run_case
from tests.test_gpu_decode_fused import _run_both, _setup
from tests.test_gpu_prefill_attention import check, run_prefill

pytestmark = pytest.mark.gpu

LENS = [1, 15, 16, 17, 31, 32, 33, 100, 129, 300, 513]


@pytest.mark.parametrize("D", [24, 32, 48, 80, 96, 112])
@pytest.mark.parametrize("paged", [False, True])
def test_decode_bf16_tile_head_dims(D, paged):
    got, ref, _ = run_case(LENS, Hq=12, Hkv=4, D=D, paged=paged, seed=D + 3 * paged)
    assert_close(got, ref)


@pytest.mark.parametrize("D", [32, 48, 80, 96])
@pytest.mark.parametrize("paged", [False, True])
def test_decode_fp8_tile_head_dims(D, paged):
    got, ref, _ = run_case([1, 16, 33, 250, 700], Hq=10, Hkv=2, D=D, paged=paged, fp8=True, seed=11 + D)
    assert_close(got, ref)


@pytest.mark.parametrize("D", [24, 48, 96])
@pytest.mark.parametrize("split", [128, 512])
def test_decode_fixed_split_padded(D, split):
    got, ref, _ = run_case([1, 100, 700, 1500], Hq=8, Hkv=2, D=D, paged=True, split_tokens=split, seed=D + split)
    assert_close(got, ref)


@pytest.mark.parametrize("G", [3, 5, 6, 7, 12])
@pytest.mark.parametrize("D", [32, 64, 128])
def test_decode_non_power_of_two_groups(G, D):
    Hkv = 2
    got, ref, _ = run_case([40, 257, 600, 1], Hq=Hkv * G, Hkv=Hkv, D=D, paged=True, seed=G * D)
    assert_close(got, ref)


@pytest.mark.parametrize("D,kind", [(2, "bf16"), (6, "bf16"), (36, "bf16"), (50, "bf16"), (126, "bf16"),
                                    (24, "fp8"), (40, "fp8"), (56, "fp8"), (24, "f32"), (32, "f32"),
                                    (48, "f32"), (100, "f32")])
@pytest.mark.parametrize("paged", [False, True])
def test_decode_valu_head_dims(D, kind, paged):
    """Head dims off the MFMA tiles (and fp32 caches): the VALU kernel."""
    got, ref, _ = run_case([1, 17, 64, 300], Hq=6, Hkv=2, D=D, paged=paged, fp8=kind == "fp8", f32=kind == "f32",
                           seed=D + paged)
    if kind == "f32":
        assert np.allclose(got, ref, rtol=1e-4, atol=1e-5)
    else:
        assert_close(got, ref)


# fp8 MFMA tiles need head_dim % 16 == 0 (fp8 D 24 is refused below)
@pytest.mark.parametrize("D,kv", [(24, "bf16"), (32, "bf16"), (48, "bf16"), (96, "bf16"),
                                  (32, "fp8"), (48, "fp8"), (96, "fp8")])
@pytest.mark.parametrize("from_partials", [False, True])
def test_fused_step_head_dims(D, kv, from_partials):
    lens = [31, 32, 1, 77, 250, 16, 600]
    Hq, Hkv = 10, 2  # G = 5
    layer, table, g = _setup(kv, True, D, Hq, Hkv, lens, seed=D)
    _run_both(layer, table, g, Hq, from_partials)


def test_fused_step_refuses_fp8_rows_off_the_tiles():
    """fp8 rows of 24 codes are not whole 16-byte fragments: the fused step
    (MFMA kernels only) refuses them with the library's message."""
    from tinytron_amd import ops

    layer, table, g = _setup("fp8", True, 24, 10, 2, [31, 32, 1], seed=3)
    B = 3
    q1 = torch.randn(B, 10, 24, generator=g).to(torch.bfloat16).cuda()
    k1 = torch.randn(B, 2, 24, generator=g).to(torch.bfloat16).cuda()
    with pytest.raises(ValueError, match="head_dim"):
        ops.decode_attention_append(table, layer._lens_dev[layer._cur], layer.layout, 40, q=q1, k=k1, v=k1)


@pytest.mark.parametrize("D,fp8", [(24, False), (32, False), (48, False), (96, False),
                                   (32, True), (48, True), (96, True)])
@pytest.mark.parametrize("G", [3, 5])
def test_prefill_head_dims(D, G, fp8):
    got, ref, new = run_prefill([0, 5, 40, 0], [33, 1, 70, 16], Hq=2 * G, Hkv=2, D=D, fp8=fp8, seed=D * G + fp8)
    check(got, ref, new)
