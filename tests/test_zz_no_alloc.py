"""rrl_fused_logprob_policy_noalloc (records in a static device array) against
rrl_fused_logprob_policy (records in a caller workspace), through the C ABI.

Both run the same kernels on the same inputs, so every output must be
bit-identical: log-probs, log-sum-exps, dlogits and the status word.  Two
calls in a row, the second on a smaller batch, show that the array's leftover
contents from a larger call do not leak into a later one.  Sizes beyond the
array's capacity are rejected on the host before any device work.
"""

from __future__ import annotations

import ctypes

import pytest
import torch

from rosellm_amd import _native as nat
from rosellm_amd.roserlhf import losses as L

pytestmark = pytest.mark.gpu


def _inputs(seed, B, T, V, dtype, device):
    g = torch.Generator().manual_seed(seed)
    x = (torch.randn(B, T, V, generator=g) * 3.0).to(dtype)
    tgt = torch.randint(0, V, (B, T), generator=g)
    old = torch.randn(B, T, generator=g) * 0.1 - 10.0
    adv = torch.randn(B, generator=g)[:, None].expand(B, T)
    lengths = torch.randint(1, T + 1, (B,), generator=g)
    mask = torch.arange(T)[None, :] < lengths[:, None]
    return [t.to(device) for t in (x, tgt, old, adv, mask)]


def _call(noalloc, params, x, tgt, old, adv, mask):
    dev = x.device
    B, T, V = x.shape
    acc_code = nat.F32
    stream = nat.stream_ptr(dev)
    pref = L.ctypes_ref(params)
    lib = nat.lib()
    coef = torch.empty(B, dtype=torch.float32, device=dev)
    ws = torch.empty(lib.rrl_policy_workspace_bytes(B, acc_code), dtype=torch.uint8, device=dev)
    logp = torch.full((B * T,), float("nan"), dtype=torch.float32, device=dev)
    lse = torch.full((B * T,), float("nan"), dtype=torch.float32, device=dev)
    dl = torch.full_like(x, float("nan"))
    status = torch.zeros(1, dtype=torch.int32, device=dev)
    tv, _a = nat.rows_view(tgt, B, T)
    ov, _b = nat.rows_view(old, B, T)
    av, _c = nat.rows_view(adv, B, T)
    mv, _d = nat.rows_view(mask, B, T)
    nat.call("rrl_policy_row_coef", pref, B, T, mv, acc_code, coef.data_ptr(), ws.data_ptr(),
             status.data_ptr(), stream)
    dt = nat.dtype_code(x.dtype)
    if noalloc:
        nat.call("rrl_fused_logprob_policy_noalloc", pref, x.data_ptr(), dt, B, T, V, T * V, V,
                 tv, ov, av, mv, coef.data_ptr(), logp.data_ptr(), lse.data_ptr(),
                 dl.data_ptr(), dt, T * V, V, status.data_ptr(), stream)
    else:
        records = torch.empty(lib.rrl_fused_records_bytes(B, T), dtype=torch.uint8, device=dev)
        nat.call("rrl_fused_logprob_policy", pref, x.data_ptr(), dt, B, T, V, T * V, V, tv, ov,
                 av, mv, coef.data_ptr(), records.data_ptr(), logp.data_ptr(), lse.data_ptr(),
                 dl.data_ptr(), dt, T * V, V, status.data_ptr(), stream)
    torch.cuda.synchronize()
    return logp, lse, dl, int(status.item())


# The second case is smaller than the first in every dimension; the third
# runs the float32 logits of config 1's vocabulary.
CASES = [
    (301, 8, 1000, 32768, torch.bfloat16, "clipped"),
    (302, 3, 257, 4104, torch.bfloat16, "sapo"),
    (303, 2, 128, 50257, torch.float32, "clipped"),
]


def test_noalloc_matches_workspace_entry_point(device):
    for seed, B, T, V, dtype, objective in CASES:
        print(f"[noalloc] B={B} T={T} V={V} {dtype} {objective}", flush=True)
        x, tgt, old, adv, mask = _inputs(seed, B, T, V, dtype, device)
        if objective == "clipped":
            p = L._params(nat.OBJ_PPO, clip_low=0.2, clip_high=0.28)
        else:
            p = L._params(nat.OBJ_SAPO, tau_positive=1.0, tau_negative=1.05)
        want = _call(False, p, x, tgt, old, adv, mask)
        got = _call(True, p, x, tgt, old, adv, mask)
        assert got[3] == want[3] == 0, (got[3], want[3])
        assert torch.equal(got[0], want[0]), "log-probs differ"
        assert torch.equal(got[1], want[1]), "log-sum-exps differ"
        assert torch.equal(got[2], want[2]), "dlogits differ"
        assert not torch.isnan(got[2]).any()


def test_noalloc_rejects_batches_beyond_its_scratch():
    lib = nat.load()
    p = L._params(nat.OBJ_PPO, clip_low=0.2, clip_high=0.2)
    nv = nat.NONE_VIEW
    tv = nat.RrlView(None, nat.I64, 1, 1)
    too_many = (1 << 20) + 1
    rc = lib.rrl_fused_logprob_policy_noalloc(ctypes.byref(p), None, nat.BF16, 1, too_many, 8,
                                              8 * too_many, 8, tv, nv, nv, nv, None, None, None,
                                              None, nat.BF16, 8 * too_many, 8, None, None)
    assert rc == -1
    assert b"exceeds the static scratch" in lib.rrl_last_error()


class _Buffers:
    """Every device buffer of one noalloc call, allocated up front, so that a
    call (or its capture) allocates nothing through the test either."""

    def __init__(self, params, x, tgt, old, adv, mask):
        dev = x.device
        B, T, V = x.shape
        self.params, self.x = params, x
        self.B, self.T, self.V = B, T, V
        self.coef = torch.empty(B, dtype=torch.float32, device=dev)
        self.ws = torch.empty(nat.lib().rrl_policy_workspace_bytes(B, nat.F32),
                              dtype=torch.uint8, device=dev)
        self.logp = torch.full((B * T,), float("nan"), dtype=torch.float32, device=dev)
        self.lse = torch.full((B * T,), float("nan"), dtype=torch.float32, device=dev)
        self.dl = torch.full_like(x, float("nan"))
        self.status = torch.zeros(1, dtype=torch.int32, device=dev)
        self.keep = (tgt, old, adv, mask)
        self.tv, _a = nat.rows_view(tgt, B, T)
        self.ov, _b = nat.rows_view(old, B, T)
        self.av, _c = nat.rows_view(adv, B, T)
        self.mv, _d = nat.rows_view(mask, B, T)
        self.views_keep = (_a, _b, _c, _d)

    def launch(self):
        """Row coefficients, then the noalloc sweep, on torch's current stream
        (the capture stream inside torch.cuda.graph)."""

        B, T, V = self.B, self.T, self.V
        stream = torch.cuda.current_stream(self.x.device).cuda_stream
        pref = L.ctypes_ref(self.params)
        dt = nat.dtype_code(self.x.dtype)
        nat.call("rrl_policy_row_coef", pref, B, T, self.mv, nat.F32, self.coef.data_ptr(),
                 self.ws.data_ptr(), self.status.data_ptr(), stream)
        nat.call("rrl_fused_logprob_policy_noalloc", pref, self.x.data_ptr(), dt, B, T, V, T * V,
                 V, self.tv, self.ov, self.av, self.mv, self.coef.data_ptr(),
                 self.logp.data_ptr(), self.lse.data_ptr(), self.dl.data_ptr(), dt, T * V, V,
                 self.status.data_ptr(), stream)

    def outputs(self):
        return self.logp.clone(), self.lse.clone(), self.dl.clone(), int(self.status.item())

    def poison(self):
        self.logp.fill_(float("nan"))
        self.lse.fill_(float("nan"))
        self.dl.fill_(float("nan"))
        self.status.zero_()


def test_noalloc_allocates_no_device_memory(device):
    """After the first call on the device (which looks up the array's address),
    a call changes neither the driver's free device memory nor torch's
    allocator state."""

    seed, B, T, V, dtype, objective = CASES[0]
    print(f"[noalloc-mem] B={B} T={T} V={V} {dtype}", flush=True)
    x, tgt, old, adv, mask = _inputs(seed, B, T, V, dtype, device)
    bufs = _Buffers(L._params(nat.OBJ_PPO, clip_low=0.2, clip_high=0.28), x, tgt, old, adv,
                    mask)
    bufs.launch()
    torch.cuda.synchronize()
    want = bufs.outputs()
    bufs.poison()
    torch.cuda.synchronize()
    free0, _total = torch.cuda.mem_get_info(device)
    alloc0 = torch.cuda.memory_allocated(device)
    reserved0 = torch.cuda.memory_reserved(device)
    bufs.launch()
    torch.cuda.synchronize()
    free1, _total = torch.cuda.mem_get_info(device)
    assert free1 == free0, f"free device memory moved by {free0 - free1} bytes"
    assert torch.cuda.memory_allocated(device) == alloc0
    assert torch.cuda.memory_reserved(device) == reserved0
    got = bufs.outputs()
    assert got[3] == want[3] == 0
    for a, b in zip(got[:3], want[:3]):
        assert torch.equal(a, b)


def test_noalloc_under_graph_capture(device):
    """The warmed-up call captured in a HIP graph (torch.cuda.graph): three
    replays, with eager work and synchronisations between them, each
    bit-identical to the uncaptured call."""

    seed, B, T, V, dtype, objective = CASES[1]
    print(f"[noalloc-graph] B={B} T={T} V={V} {dtype}", flush=True)
    x, tgt, old, adv, mask = _inputs(seed, B, T, V, dtype, device)
    bufs = _Buffers(L._params(nat.OBJ_SAPO, tau_positive=1.0, tau_negative=1.05), x, tgt, old,
                    adv, mask)
    bufs.launch()
    torch.cuda.synchronize()
    want = bufs.outputs()
    assert want[3] == 0 and not torch.isnan(want[2]).any()
    bufs.poison()
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        bufs.launch()
    torch.cuda.synchronize()
    for rep in range(3):
        bufs.poison()  # eager fill kernels between the replays
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        got = bufs.outputs()
        print(f"[noalloc-graph] replay {rep}", flush=True)
        assert got[3] == 0, got[3]
        for a, b, what in zip(got[:3], want[:3], ("log-probs", "lse", "dlogits")):
            assert torch.equal(a, b), f"replay {rep}: {what} differ from the uncaptured call"
