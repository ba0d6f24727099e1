"""z2h_model_moe_forward_noalloc (one MoE layer on a model alone, every intermediate buffer carved from
the library's static device scratch, no allocation) against the existing entry point that takes its
buffers from a context (z2h_moe_forward_device, through z2h_moe_forward): bit-identical outputs and
router state on two calls in a row, the second with fewer tokens (the scratch keeps the first call's
contents), for Q4_K experts (fused gate/up + SwiGLU GEMVs, and from 65 tokens the sorted route table
and the int8 MFMA GEMMs), Q6_K and Q8_0 experts (the m16 GEMVs) and F16 experts (the fp16 MFMA GEMMs);
a call whose buffers exceed the scratch is refused before any launch."""
import dataclasses

import numpy as np
import pytest
import torch

from zonos2_amd import configs, synth
from zonos2_amd.z2h import Context, Model, Z2HError

pytestmark = pytest.mark.gpu


def _dev(a):
    return torch.from_numpy(np.ascontiguousarray(a)).to("cuda:0")


# tokens per call: Q4_K adds a 96-token call (from 65 rows the wide path: k_router_down_t,
# k_router_tail<true>, k_route_sort and the k_gemm_q4k expert GEMMs, their tables in the scratch)
@pytest.mark.parametrize("bulk,calls", [(configs.Q4_K, (96, 40, 7)), (configs.Q6_K, (40, 7)), (configs.Q8_0, (40, 7)),
                                        (configs.F16, (24, 7))], ids=["q4_k", "q6_k", "q8_0", "f16"])
def test_noalloc_moe_layer_matches_the_context_entry_point(bulk, calls):
    cfg, wl = configs.C2()
    cfg = dataclasses.replace(cfg, bulk=bulk)
    model = synth.generate_model(cfg, 42)
    m = Model(cfg.hparams(), model)
    ctx = Context(None, 128, 256, model=m, max_rows=128)
    ctx.set_capture(True)
    rd = cfg.router_dim
    dev0 = torch.cuda.current_device()
    for T in calls:                                    # later calls: fewer tokens, scratch holds the earlier data
        print(f"{cfg.name} T={T}", flush=True)
        x = synth.gen_normal_f32((T, cfg.n_embd), 11 + T, "inputs.noalloc")
        st = synth.gen_normal_f32((T, rd), 12 + T, "state.noalloc")
        want = ctx.moe_forward(0, x, st)
        want_state = ctx.read_capture(0, "router_state", T).reshape(T, rd)
        dx, ds, dso = _dev(x), _dev(st), torch.empty((T, rd), dtype=torch.float32, device="cuda:0")
        dout = torch.full((T, cfg.n_embd), float("nan"), dtype=torch.float32, device="cuda:0")
        torch.cuda.synchronize()
        m.moe_forward_noalloc(0, T, dx.data_ptr(), ds.data_ptr(), dso.data_ptr(), dout.data_ptr())
        torch.cuda.synchronize()
        got = dout.cpu().numpy()
        assert np.array_equal(got.view(np.uint32), want.view(np.uint32)), f"T={T}: outputs differ"
        assert np.array_equal(dso.cpu().numpy().view(np.uint32), want_state.view(np.uint32)), f"T={T}: router state differs"
        assert torch.cuda.current_device() == dev0
    # state kept in the scratch (d_state_out NULL): same outputs
    dout2 = torch.empty((7, cfg.n_embd), dtype=torch.float32, device="cuda:0")
    m.moe_forward_noalloc(0, 7, dx.data_ptr(), ds.data_ptr(), 0, dout2.data_ptr())
    torch.cuda.synchronize()
    assert np.array_equal(dout2.cpu().numpy().view(np.uint32), want.view(np.uint32))
    # too many tokens for the scratch (or for the route lists): refused before any launch
    big = torch.zeros((256, cfg.n_embd), dtype=torch.float32, device="cuda:0")
    with pytest.raises(Z2HError) as e:
        m.moe_forward_noalloc(0, 256, big.data_ptr(), 0, 0, big.data_ptr())
    assert "n_tokens out of range" in str(e.value) or "scratch" in str(e.value)
    ctx.close()
    m.close()
