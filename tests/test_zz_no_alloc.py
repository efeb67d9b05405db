"""burnext_moe_forward_noalloc (the forward on the library's fixed per-GPU scratch) against
burnext_moe_forward with a caller workspace, through the C ABI: bit-identical outputs on two calls
in a row, the second with a smaller batch, and a clear error for a batch beyond the scratch."""
import numpy as np
import pytest

torch = pytest.importorskip("torch")

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def M():
    if not torch.cuda.is_available():
        pytest.skip("no HIP device")
    from burnext_amd import moe
    return moe


@pytest.mark.parametrize("D,F,E,K,n1,n2,dtype,fused", [
    (2880, 2880, 32, 4, 8, 3, "bf16", False),    # 20B decode, then a smaller batch
    (2880, 2880, 128, 4, 64, 1, "bf16", False),  # 120B: mid-size GEMV batch, then one token (K-part path)
    (256, 256, 4, 2, 16, 5, "f32", False),
    (2880, 2880, 32, 4, 16, 2, "bf16", True),    # the opt-in fused experts kernel, slices in the scratch
])
def test_forward_noalloc_matches_forward(M, D, F, E, K, n1, n2, dtype, fused):
    from burnext_amd import _native as N, synth
    flags = N.FORWARD_DEFAULT | (N.FUSED_EXPERTS if fused else 0)
    print(f"noalloc D={D} E={E} n={n1} then {n2} {dtype} fused={fused}", flush=True)
    L = synth.make_layer(D, F, E, K, seed=31, dtype=dtype, with_gamma=True)
    layer = M.MoeLayer(L)
    for n, seed in ((n1, 1), (n2, 2)):
        x = M.to_device_x(synth.make_tokens(n, D, seed=seed, dtype=dtype), dtype)
        y_ref = layer.forward(x, flags=flags)
        y = torch.full_like(x, float("nan"))
        layer.forward_noalloc(x, out=y, flags=flags)
        torch.cuda.synchronize()
        iv = torch.int16 if dtype == "bf16" else torch.int32
        assert torch.equal(y.view(iv), y_ref.view(iv)), f"n={n}"
    layer.close()


def test_forward_noalloc_rejects_batches_beyond_scratch(M):
    from burnext_amd import _native as N, synth
    L = synth.make_layer(2880, 2880, 32, 4, seed=0, dtype="bf16")
    layer = M.MoeLayer(L)
    n = 4096
    assert layer.workspace_size(n) > 16 << 20
    x = torch.zeros((n, 2880), dtype=torch.bfloat16, device="cuda")
    y = torch.empty_like(x)
    with pytest.raises(N.BurnextError) as ei:
        layer.forward_noalloc(x, out=y)
    assert ei.value.status == N.BURNEXT_UNSUPPORTED and "scratch" in str(ei.value)
    layer.close()
