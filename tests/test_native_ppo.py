"""The PPO integration's host-side pieces (no GPU): GAE against the
reference's known answers (tests/test_native_ppo.py:32-73) and its closed
forms, the action tables, config validation, checkpoint round trip and the
model's shape and initialisation."""

from __future__ import annotations

import numpy as np
import pytest
import torch

from nesle_amd import actions as A
from nesle_amd import native_ppo as P


def test_gae_known_answer_discounted_returns_when_values_zero():
    rewards = torch.tensor([[1.0, 1.0], [1.0, 2.0], [1.0, 3.0]])
    z = torch.zeros_like(rewards)
    _, returns = P.compute_gae(rewards, z, z, torch.zeros(2), torch.zeros(2), gamma=0.5, gae_lambda=1.0)
    np.testing.assert_allclose(returns.numpy(), [[1.75, 2.75], [1.5, 3.5], [1.0, 3.0]], rtol=1e-6)


def test_gae_known_answer_stops_at_done_boundary():
    rewards = torch.tensor([[1.0], [1.0], [10.0]])
    dones = torch.tensor([[0.0], [0.0], [1.0]])
    z = torch.zeros_like(rewards)
    _, returns = P.compute_gae(rewards, dones, z, torch.zeros(1), torch.zeros(1), gamma=0.9, gae_lambda=1.0)
    np.testing.assert_allclose(returns.numpy(), [[1.9], [1.0], [10.0]], rtol=1e-6)


def test_gae_closed_forms():
    g = torch.Generator().manual_seed(3)
    T, N, gamma = 9, 5, 0.97
    r, v = torch.rand(T, N, generator=g), torch.rand(T, N, generator=g)
    nv = torch.rand(N, generator=g)
    zero = torch.zeros(T, N)
    # lambda = 0: one-step TD errors.
    adv0, _ = P.compute_gae(r, zero, v, torch.zeros(N), nv, gamma, 0.0)
    nxt = torch.cat([v[1:], nv[None]], 0)
    torch.testing.assert_close(adv0, r + gamma * nxt - v)
    # lambda = 1, no episode ends: returns are the discounted sum bootstrapped by next_value.
    _, ret1 = P.compute_gae(r, zero, v, torch.zeros(N), nv, gamma, 1.0)
    want = torch.empty(T, N)
    acc = nv.clone()
    for t in range(T - 1, -1, -1):
        acc = r[t] + gamma * acc
        want[t] = acc
    torch.testing.assert_close(ret1, want)
    # An episode start at t cuts the bootstrap from t onwards.
    d = zero.clone()
    d[4] = 1.0
    adv, _ = P.compute_gae(r, d, v, torch.zeros(N), nv, gamma, 1.0)
    torch.testing.assert_close(adv[3], r[3] - v[3])


def test_action_tables_known_answers():
    # A=bit0 B=1 SELECT=2 START=3 UP=4 DOWN=5 LEFT=6 RIGHT=7
    assert A.COMPLEX_MOVEMENT_MASKS == (0x00, 0x80, 0x81, 0x82, 0x83, 0x01, 0x40, 0x41, 0x42, 0x43, 0x20, 0x10)
    assert A.SIMPLE_MOVEMENT_WITH_START_MASKS == (0x08, 0x00, 0x80, 0x81, 0x82, 0x83, 0x01, 0x40)
    assert A.RIGHT_ONLY_MASKS == (0x00, 0x80, 0x81, 0x82, 0x83)
    assert A.MARIO_MOVEMENT_MASKS == (0x00, 0x80, 0x82, 0x81, 0x83, 0x01, 0x03, 0x40, 0x41, 0x20, 0xA0)
    assert A.action_masks("complex") == A.COMPLEX_MOVEMENT_MASKS
    assert A.action_masks("raw") == tuple(range(256))
    assert A.action_masks([0x1FF, 3]) == (0xFF, 3)
    with pytest.raises(ValueError):
        A.encode_action(["jump"])
    with pytest.raises(ValueError):
        A.action_masks("sideways")


def test_rollout_smaller_than_batch_is_rejected_before_any_device_work():
    cfg = P.NativePPOConfig("none.nes", num_envs=8, n_steps=4, batch_size=64)
    with pytest.raises(ValueError, match="batch_size"):
        P.train_native_ppo(cfg)


def test_model_shapes_and_init():
    for init in ("orthogonal", "xavier"):
        torch.manual_seed(0)
        m = P._make_model(2048, 12, 256, init, torch.device("cpu"))
        logits, value = m(torch.randint(0, 256, (5, 2048), dtype=torch.uint8))
        assert logits.shape == (5, 12) and value.shape == (5,)
        w = m.net[0].weight.detach()
        if init == "orthogonal":   # rows orthonormal up to the gain sqrt(2)
            gram = w @ w.T / 2.0
            torch.testing.assert_close(gram, torch.eye(256), atol=1e-4, rtol=0)
        else:                      # Xavier uniform bound sqrt(2) * sqrt(6 / (fan_in + fan_out))
            assert float(w.abs().max()) <= np.sqrt(2.0) * np.sqrt(6.0 / (2048 + 256)) + 1e-6
        assert float(m.actor.bias.detach().abs().max()) == 0.0


def test_checkpoint_round_trip_restores_rng_and_weights(tmp_path):
    model = torch.nn.Linear(4, 2)
    opt = torch.optim.Adam(model.parameters(), lr=1e-3)
    cfg = P.NativePPOConfig("dummy.nes")
    torch.manual_seed(42)
    np.random.seed(42)
    path = tmp_path / "nested" / "ckpt.pt"
    P._save_checkpoint(str(path), model, opt, cfg, global_step=1234)
    a_t, a_n = torch.rand(5), np.random.rand(5)
    model2 = torch.nn.Linear(4, 2)
    opt2 = torch.optim.Adam(model2.parameters(), lr=1e-3)
    assert P._load_checkpoint(str(path), model2, opt2) == 1234
    torch.testing.assert_close(torch.rand(5), a_t)
    np.testing.assert_allclose(np.random.rand(5), a_n)
    torch.testing.assert_close(model2.weight, model.weight)


def test_checkpoint_restores_adam_to_the_trainer_configuration(tmp_path):
    """A checkpoint keeps the flags its Adam was saved with (the reference's
    plain Adam: host step counters); the trainer sets fused and capturable
    again after loading and moves the step counters to the parameters'
    device as float32."""
    torch.manual_seed(0)
    model = P._make_model(2048, 7, 32, "orthogonal", torch.device("cpu"))
    opt = torch.optim.Adam(model.parameters(), lr=1e-3, eps=1e-5)
    logits, value = model(torch.randint(0, 256, (4, 2048), dtype=torch.uint8))
    (logits.sum() + value.sum()).backward()
    opt.step()
    path = tmp_path / "ckpt.pt"
    P._save_checkpoint(str(path), model, opt, P.NativePPOConfig("rom.nes"), 77)
    opt2 = torch.optim.Adam(model.parameters(), lr=1e-3, eps=1e-5, capturable=True, fused=True)
    assert P._load_checkpoint(str(path), model, opt2) == 77
    assert all(not g["capturable"] and not g["fused"] for g in opt2.param_groups)      # the saved flags
    P._configure_adam(torch, opt2)
    assert all(g["capturable"] and g["fused"] for g in opt2.param_groups)
    for p in model.parameters():
        step = opt2.state[p]["step"]
        assert step.dtype == torch.float32 and step.device == p.device and float(step) == 1.0
    for p in model.parameters():
        p.grad = torch.ones_like(p)
    opt2.step()
    assert all(float(opt2.state[p]["step"]) == 2.0 for p in model.parameters())


def test_ppo_head_refuses_host_tensors_before_any_launch():
    """The HIP loss head takes device pointers only: host tensors, wrong
    dtypes or shapes are rejected in Python, and the C entry point rejects
    bad sizes and null pointers before it launches anything."""
    from nesle_amd import abi

    n, a = 8, 5
    args = [torch.zeros(n, a), torch.zeros(n), torch.zeros(n, dtype=torch.int64), torch.zeros(n), torch.zeros(n),
            torch.zeros(n)]
    with pytest.raises(ValueError, match="GPU tensor"):
        P.ppo_head_loss(*args, 0.1, 0.01, 0.5)
    L = abi.lib()
    assert L.nesle_ppo_head_scratch_floats(8192) == 2 + 4 * 32
    assert L.nesle_ppo_head_scratch_floats(257) == 2 + 4 * 2
    for batch, actions in ((0, 12), (16, 0), (16, 1025)):
        assert L.nesle_ppo_head(*([None] * 6), batch, actions, 0.1, 0.01, 0.5, *([None] * 7)) == abi.EINVAL
        assert b"num_actions" in L.nesle_last_error()
    assert L.nesle_ppo_head(*([None] * 6), 16, 12, 0.1, 0.01, 0.5, *([None] * 7)) == abi.EINVAL
    assert b"null" in L.nesle_last_error()


def test_explained_variance_closed_forms():
    g = torch.Generator().manual_seed(5)
    ret = torch.rand(1000, generator=g)
    assert P._explained_variance(ret, ret) == 1.0                     # perfect prediction
    assert abs(P._explained_variance(torch.zeros(1000), ret)) < 1e-6     # predicting nothing
    mean = torch.full((1000,), float(ret.mean()))
    assert abs(P._explained_variance(mean, ret)) < 1e-5                 # a constant explains no variance
    half = ret * 0.5
    want = 1.0 - float((ret - half).var()) / float(ret.var())          # Var(r/2) / Var(r) = 1/4
    assert abs(P._explained_variance(half, ret) - want) < 1e-6 and abs(want - 0.75) < 1e-6
    assert np.isnan(P._explained_variance(torch.rand(10), torch.ones(10)))


def test_checkpoint_without_model_or_optimizer_is_refused(tmp_path):
    path = tmp_path / "other.pt"
    torch.save({"model": {}, "global_step": 3}, path)
    model = torch.nn.Linear(2, 2)
    with pytest.raises(ValueError, match="checkpoint"):
        P._load_checkpoint(str(path), model, torch.optim.Adam(model.parameters()))
    assert P._load_checkpoint(str(tmp_path / "missing.pt"), model, torch.optim.Adam(model.parameters())) == 0


def test_checkpoint_keeps_the_reference_key_names(tmp_path):
    """Top-level keys as the reference trainer writes them (native_ppo.py:
    319-368), every value loadable with weights_only=True."""
    model = torch.nn.Linear(3, 2)
    opt = torch.optim.Adam(model.parameters())
    path = tmp_path / "ckpt.pt"
    P._save_checkpoint(str(path), model, opt, P.NativePPOConfig("rom.nes"), 5)
    ckpt = torch.load(path, weights_only=True)
    assert {"model", "optimizer", "config", "global_step", "torch_rng_state", "numpy_rng_state"} <= set(ckpt)
    name, keys, pos, has_gauss, cached = ckpt["numpy_rng_state"]
    assert name == "MT19937" and keys.shape == (624,) and 0 <= pos <= 624
    assert ckpt["config"]["rom_path"] == "rom.nes" and ckpt["global_step"] == 5


def test_checkpoint_of_the_earlier_layout_still_loads(tmp_path):
    """Files of the layout that kept the RNG states under one "rng" entry
    (format nesle_amd.native_ppo/1) resume: weights, step count and RNGs."""
    model = torch.nn.Linear(4, 2)
    opt = torch.optim.Adam(model.parameters())
    np.random.seed(9)
    torch.manual_seed(9)
    mt = np.random.get_state(legacy=False)
    old = {"format": "nesle_amd.native_ppo/1", "global_step": 321, "config": {}, "model": model.state_dict(),
           "optimizer": opt.state_dict(),
           "rng": {"torch": torch.get_rng_state(), "numpy_key": torch.from_numpy(mt["state"]["key"].astype(np.int64)),
                   "numpy_pos": int(mt["state"]["pos"]), "numpy_has_gauss": int(mt["has_gauss"]),
                   "numpy_gauss": float(mt["gauss"])}}
    path = tmp_path / "old.pt"
    torch.save(old, path)
    a_t, a_n = torch.rand(3), np.random.rand(3)
    model2 = torch.nn.Linear(4, 2)
    assert P._load_checkpoint(str(path), model2, torch.optim.Adam(model2.parameters())) == 321
    torch.testing.assert_close(model2.weight, model.weight)
    torch.testing.assert_close(torch.rand(3), a_t)
    np.testing.assert_allclose(np.random.rand(3), a_n)
