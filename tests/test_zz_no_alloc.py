"""nesle_ppo_head_static (include/nesle_ppo.h), the loss head entry point that
allocates nothing: through the C ABI, two calls in a row (the second with a
smaller minibatch) give bit-identical loss, clip fraction, accumulator and
gradients to nesle_ppo_head with a caller-provided workspace on the same
inputs, and a minibatch beyond the static scratch is refused before any
launch."""

from __future__ import annotations

import ctypes

import pytest

from tests.helpers import say

pytestmark = pytest.mark.gpu


def _inputs(torch, n: int, a: int, seed: int):
    g = torch.Generator(device="cuda").manual_seed(seed)
    dev = torch.device("cuda")
    logits = torch.randn(n, a, generator=g, device=dev)
    value = torch.randn(n, generator=g, device=dev)
    actions = torch.randint(0, a, (n,), generator=g, device=dev)
    old_logprob = torch.log_softmax(logits + 0.3 * torch.randn(n, a, generator=g, device=dev), dim=1)[
        torch.arange(n, device=dev), actions].contiguous()
    adv = torch.randn(n, generator=g, device=dev)
    ret = torch.randn(n, generator=g, device=dev)
    return logits, value, actions, old_logprob, adv, ret


def _run(torch, L, static: bool, args, clip=0.1, ent=0.01, vf=0.5, accum_start=(1.0, 2.0)):
    logits, value, actions, old_logprob, adv, ret = args
    n, a = logits.shape
    dlogits = torch.full_like(logits, float("nan"))
    dvalue = torch.full_like(value, float("nan"))
    loss = torch.full((), float("nan"), device="cuda")
    clipfrac = torch.full((), float("nan"), device="cuda")
    accum = torch.tensor(accum_start, dtype=torch.float32, device="cuda")
    stream = torch.cuda.current_stream().cuda_stream
    ins = [t.data_ptr() for t in (logits, value, actions, old_logprob, adv, ret)]
    if static:
        rc = L.nesle_ppo_head_static(*ins, n, a, clip, ent, vf, dlogits.data_ptr(), dvalue.data_ptr(),
                                     loss.data_ptr(), clipfrac.data_ptr(), accum.data_ptr(), stream)
    else:
        work = torch.empty(int(L.nesle_ppo_head_scratch_floats(n)), dtype=torch.float32, device="cuda")
        rc = L.nesle_ppo_head(*ins, n, a, clip, ent, vf, dlogits.data_ptr(), dvalue.data_ptr(), work.data_ptr(),
                              loss.data_ptr(), clipfrac.data_ptr(), accum.data_ptr(), stream)
    assert rc == 0, L.nesle_last_error()
    torch.cuda.synchronize()
    return dlogits, dvalue, loss, clipfrac, accum


def test_static_head_matches_workspace_head_on_two_calls():
    import torch

    from nesle_amd import abi

    L = abi.lib()
    for n, a, seed in ((8192, 12, 1), (300, 7, 2)):
        say(f"[gpu] no-alloc loss head: batch={n} actions={a}")
        args = _inputs(torch, n, a, seed)
        want = _run(torch, L, False, args)
        got = _run(torch, L, True, args)
        for w, g, name in zip(want, got, ("dlogits", "dvalue", "loss", "clipfrac", "accum")):
            assert torch.equal(w, g), f"batch {n}: {name} differs"
        assert torch.isfinite(got[2]) and float(got[3]) > 0.0


def test_static_head_refuses_oversized_minibatch():
    from nesle_amd import abi

    L = abi.lib()
    big = 1048576 + 1
    rc = L.nesle_ppo_head_static(*([ctypes.c_void_p(8)] * 6), big, 12, 0.1, 0.01, 0.5, ctypes.c_void_p(8),
                                 ctypes.c_void_p(8), ctypes.c_void_p(8), ctypes.c_void_p(8), None, None)
    assert rc == abi.EINVAL
    assert b"exceeds the static scratch" in L.nesle_last_error()
