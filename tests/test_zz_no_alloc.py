"""tlm_hip_moe_layer_noalloc (no counterpart in the reference; for callers
that cannot allocate): the MoE block with its workspace in the library's
static per-device array.  Through the C ABI, against tlm_hip_moe_layer with a
caller workspace, bit for bit (residual, routing ids and weights), on two
calls in a row - the Qwen3-30B-A3B-shape block, then a smaller one, so the
second call runs on the array the first left behind - and a block whose
workspace exceeds the array is refused with TLM_HIP_ERANGE before any launch."""
import ctypes as C

import numpy as np
import pytest
import torch

import oracle
from tests.synth import build_moe_case

pytestmark = pytest.mark.gpu


def noalloc(block, h):
    from tierlm_amd._lib import lib
    from tierlm_amd.quant import stream
    ids = torch.full_like(block.ids, -1)
    w = torch.full_like(block.w, -1.0)
    rc = lib.tlm_hip_moe_layer_noalloc(C.byref(block.desc), C.c_void_p(h.data_ptr()), C.c_void_p(ids.data_ptr()),
                                       C.c_void_p(w.data_ptr()), stream())
    return rc, ids, w


def same_bits(a, b):
    return np.array_equal(a.cpu().numpy().view(np.uint32), b.cpu().numpy().view(np.uint32))


def test_noalloc_equals_workspace_entry(hip, dev):
    big = build_moe_case(D=2048, de=768, E=128, k=8, ds=0, expert_dt=oracle.Q6_K, seed=5, device=dev,
                         weights="random_codes")
    small = build_moe_case(D=512, de=256, E=32, k=4, ds=256, expert_dt=oracle.Q6_K, shared_dt=oracle.Q8_0,
                           seed=21, device=dev)
    for case in (big, small):
        h0 = torch.from_numpy(case.h0.copy()).to(dev)
        ref_h = h0.clone()
        case.block(ref_h)
        got_h = h0.clone()
        rc, ids, w = noalloc(case.block, got_h)
        torch.cuda.synchronize()
        assert rc == 0
        assert same_bits(got_h, ref_h)
        assert torch.equal(ids[:case.k], case.block.ids[:case.k])
        assert same_bits(w[:case.k], case.block.w[:case.k])


def test_noalloc_refuses_oversized_workspace(hip, dev):
    from tierlm_amd._lib import TLM_HIP_ERANGE, MoeDesc, lib
    case = build_moe_case(D=512, de=256, E=32, k=4, ds=0, expert_dt=oracle.Q6_K, seed=22, device=dev)
    d = MoeDesc.from_buffer_copy(case.block.desc)
    d.de = 16384 * 16                     # k * de * 4 bytes of expert activations: far past the array
    assert lib.tlm_hip_moe_workspace_bytes(C.byref(d)) > (1 << 20)
    h = torch.from_numpy(case.h0.copy()).to(dev)
    rc = lib.tlm_hip_moe_layer_noalloc(C.byref(d), C.c_void_p(h.data_ptr()), None, None, None)
    assert rc == TLM_HIP_ERANGE
    torch.cuda.synchronize()
    assert np.array_equal(h.cpu().numpy(), case.h0)
