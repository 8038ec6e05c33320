"""The GPU-resident PPO loop (nesle_amd.native_ppo) on the HIP batch: every
rollout step's actions, rewards and done flags equal the oracle consoles
stepped with the same controller masks, with the snapshot auto-reset
and the episode-length timeout reset applied the same way; the update runs
and changes the policy."""

from __future__ import annotations

import math

import numpy as np
import pytest
import torch

from nesle_amd import native_ppo as P
from nesle_amd import synthrom
from oracle import oracle as O
from tests.helpers import OracleBatch, say, warm_snapshots

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("max_episode_steps", [0, 5])
def test_ppo_rollout_matches_oracle_and_update_learns(max_episode_steps):
    rom = synthrom.make_rom(5).rom
    warm = [100, 150, 200, 250]
    say(f"[gpu] ppo: snapshot bank, max_episode_steps={max_episode_steps}")
    snaps = warm_snapshots(rom, warm, seed=55)
    for i, s in enumerate(snaps):
        s[O.OFF["ram"] + synthrom.DONE_BYTE] = 1 + i
    n, T = 64, 16
    reward = dict(kind="x_delta", x_lo=synthrom.X_LO, x_hi=synthrom.X_HI, done_addr=synthrom.DONE_BYTE,
                  clip=15, time_penalty=0.25)
    cfg = P.NativePPOConfig("synthetic.nes", num_envs=n, n_steps=T, batch_size=256, update_epochs=2,
                            frameskip=4, action_space="complex", init="xavier", reward=reward,
                            total_timesteps=n * T, save_checkpoints=False, seed=3,
                            max_episode_steps=max_episode_steps)
    rec = []
    say(f"[gpu] ppo: N={n} T={T} one update")
    stats = P.train_native_ppo(cfg, rom_bytes=rom, snapshot_bytes=[bytes(s) for s in snaps],
                               record=lambda k, m, r, d: rec.append((m.cpu().numpy(), r.cpu().numpy().copy(),
                                                                     d.cpu().numpy().copy())))
    assert stats["updates"] == 1 and len(rec) == T
    assert math.isfinite(stats["log"][-1]["loss"])
    assert 0.0 < stats["emulator_s"] <= stats["wall_s"]

    levels = np.arange(n) % len(snaps)
    ob = OracleBatch(rom, list(range(n)), reward=dict(kind=1, x_lo=synthrom.X_LO, x_hi=synthrom.X_HI,
                                                      done_addr=synthrom.DONE_BYTE, clip=15, time_penalty=0.25))
    for e, c in enumerate(ob.cons):
        c.load(snaps[levels[e]])
    length = np.zeros(n, dtype=np.int64)
    ends = 0
    for k, (masks, rew, done) in enumerate(rec):
        assert set(np.unique(masks)) <= set(P._actions.COMPLEX_MOVEMENT_MASKS)
        _, want_r, want_d = ob.step(masks, 4)
        length += 1
        want_done = want_d.astype(bool)
        if max_episode_steps:
            want_done |= length >= max_episode_steps
        np.testing.assert_array_equal(rew, want_r, err_msg=f"step {k} rewards")
        np.testing.assert_array_equal(done, want_done, err_msg=f"step {k} dones")
        for e in np.nonzero(want_done)[0]:
            ob.cons[e].load(snaps[levels[e]])
        length[want_done] = 0
        ends += int(want_done.sum())
    assert ends > 0

    torch.manual_seed(cfg.seed)
    init = P._make_model(2048, 12, 256, "xavier", torch.device("cuda"))
    moved = [not torch.equal(a, b) for a, b in zip(init.parameters(), stats["model"].parameters())]
    assert all(moved)


def test_rollout_graph_replays_match_eager_rollouts():
    """With cuda_graph the rollouts after the first replay one captured HIP
    graph (policy, sampling, the C-ABI step and bookkeeping for all steps),
    and the minibatch steps after the first update replay another.  Every
    rollout replay, with the update replays and host synchronisations between
    them, equals the same rollout run eagerly (eager updates)."""
    rom = synthrom.make_rom(5).rom
    snaps = warm_snapshots(rom, [100, 150, 200, 250], seed=55)
    for i, s in enumerate(snaps):
        s[O.OFF["ram"] + synthrom.DONE_BYTE] = 2 + i
    n, T, updates = 64, 8, 4
    reward = dict(kind="x_delta", x_lo=synthrom.X_LO, x_hi=synthrom.X_HI, done_addr=synthrom.DONE_BYTE,
                  clip=15, time_penalty=0.25)
    runs, per_update = {}, {}
    for graph in (False, True):
        say(f"[gpu] ppo rollouts cuda_graph={graph}: N={n} T={T} updates={updates}")
        cfg = P.NativePPOConfig("synthetic.nes", num_envs=n, n_steps=T, batch_size=128, update_epochs=1,
                                frameskip=4, action_space="complex", init="xavier", reward=reward,
                                total_timesteps=n * T * updates, save_checkpoints=False, seed=11,
                                max_episode_steps=6, cuda_graph=graph)
        got = []
        stats = P.train_native_ppo(cfg, rom_bytes=rom, snapshot_bytes=[bytes(s) for s in snaps],
                                   on_rollout=lambda u, b: got.append(
                                       {k: (v.cpu().numpy().copy() if hasattr(v, "cpu") else v) for k, v in b.items()}))
        runs[graph] = got
        per_update[graph] = stats["per_update"]
        assert stats["graph_updates"] == (updates - 1 if graph else 0)
    assert [r["graph"] for r in runs[True]] == [False] + [True] * (updates - 1)
    assert [u["update_graph"] for u in per_update[True]] == [False] + [True] * (updates - 1)
    assert not any(u["update_graph"] for u in per_update[False])
    for u, (e, g) in enumerate(zip(runs[False], runs[True])):
        for key in ("actions", "rewards", "dones"):
            np.testing.assert_array_equal(g[key], e[key], err_msg=f"update {u + 1} {key}")
        for key in ("values", "logprobs"):
            np.testing.assert_allclose(g[key], e[key], rtol=0, atol=1e-5, err_msg=f"update {u + 1} {key}")
    assert sum(int(r["dones"].sum()) for r in runs[True]) > 0


def test_minibatch_graph_replays_match_eager_steps():
    """One captured minibatch step (gather, forward, the HIP loss head,
    backward, gradient-norm clipping, fused capturable Adam) replayed per
    minibatch, with eager work and host synchronisations between replays,
    leaves the parameters, Adam's moments and step counters and the loss
    sums equal to the same steps run eagerly, after every replay."""
    dev = torch.device("cuda")
    B, count = 512, 2048
    gen = torch.Generator().manual_seed(7)
    src = {"obs": torch.randint(0, 256, (count, 2048), dtype=torch.uint8, generator=gen).to(dev),
           "actions": torch.randint(0, 12, (count,), generator=gen).to(dev),
           "logprobs": (-3.0 * torch.rand(count, generator=gen)).to(dev),
           "advantages": torch.randn(count, generator=gen).to(dev),
           "returns": torch.randn(count, generator=gen).to(dev)}
    cfg = P.NativePPOConfig("synthetic.nes", batch_size=B)
    updaters = []
    for _ in range(2):
        torch.manual_seed(3)
        model = P._make_model(2048, 12, 256, "orthogonal", dev)
        opt = torch.optim.Adam(model.parameters(), lr=cfg.learning_rate, eps=1e-5, capturable=True, fused=True)
        updaters.append(P.MinibatchUpdate(torch, model, opt, cfg, src))
    eager, graphed = updaters
    idxs = [p[s:s + B] for p in (torch.randperm(count, generator=gen).to(dev) for _ in range(3))
            for s in range(0, count, B)]
    say(f"[gpu] ppo minibatch graph: B={B} count={count} steps={len(idxs)}")
    eager.run(idxs[0])
    graphed.run(idxs[0])
    graphed.capture()
    junk = torch.randn(512, 512, device=dev)
    worst = 0.0
    for k, idx in enumerate(idxs[1:], 1):
        eager.run(idx)
        graphed.run(idx)
        junk = torch.tanh(junk @ junk)
        torch.cuda.synchronize()
        for (name, a), b in zip(eager.model.named_parameters(), graphed.model.parameters()):
            worst = max(worst, float((a.detach() - b.detach()).abs().max()))
            torch.testing.assert_close(b, a, rtol=1e-5, atol=1e-6, msg=f"step {k} {name}")
            sa, sb = eager.optimizer.state[a], graphed.optimizer.state[b]
            for key in ("exp_avg", "exp_avg_sq", "step"):
                torch.testing.assert_close(sb[key], sa[key], rtol=1e-5, atol=1e-9, msg=f"step {k} {name} {key}")
        torch.testing.assert_close(graphed.sums, eager.sums, rtol=1e-5, atol=1e-6, msg=f"step {k} sums")
    assert graphed.graph is not None and eager.graph is None
    assert graphed.minibatches == eager.minibatches == len(idxs)
    assert float(eager.sums.abs().sum()) > 0.0
    say(f"[gpu] ppo minibatch graph: max parameter difference {worst:.3g}")


def _reference_loss(logits, value, actions, old_logprob, advantages, returns, clip, ent_coef, vf_coef):
    """The reference trainer's loss lines (native_ppo.py:546-566), float32."""
    from torch.distributions.categorical import Categorical

    dist = Categorical(logits=logits)
    newlogprob = dist.log_prob(actions)
    entropy = dist.entropy().mean()
    ratio = (newlogprob - old_logprob).exp()
    adv = (advantages - advantages.mean()) / (advantages.std() + 1e-8)
    pg_loss = torch.max(-adv * ratio, -adv * torch.clamp(ratio, 1.0 - clip, 1.0 + clip)).mean()
    value_loss = 0.5 * (value - returns).pow(2).mean()
    loss = pg_loss - ent_coef * entropy + vf_coef * value_loss
    clipfrac = ((ratio - 1.0).abs() > clip).float().mean()
    return loss, clipfrac


@pytest.mark.parametrize("n,a,spread", [(8192, 12, 0.3), (300, 256, 0.05), (1000, 7, 0.0), (2, 1, 0.2)])
def test_ppo_head_matches_the_reference_loss_and_its_gradients(n, a, spread):
    """The HIP loss head (nesle_ppo_head) against the reference's loss
    computed by PyTorch autograd in float32 on the host: loss, clip fraction,
    d loss / d logits and d loss / d value, for a loss gradient of 1 and of
    -2.5.  Rows mix ratios inside and outside the clip range (spread 0:
    every ratio exactly 1, the tie of the two surrogate terms), zero
    advantages, and batches that are not a multiple of the head's 256-row
    workgroup.  Tolerance 1e-5 relative on the loss, 1e-4 relative +
    1e-7 absolute per gradient element (float32 sums in another order)."""
    gen = torch.Generator().manual_seed(n * 7 + a)
    logits = 3.0 * torch.randn(n, a, generator=gen)
    value = torch.randn(n, generator=gen)
    actions = torch.randint(0, a, (n,), generator=gen)
    logp = torch.log_softmax(logits, dim=-1).gather(1, actions[:, None]).squeeze(1)
    old_logprob = logp + spread * torch.randn(n, generator=gen)
    if spread == 0.0:
        old_logprob = logp.clone()
    advantages = torch.randn(n, generator=gen)
    advantages[::5] = 0.0
    returns = torch.randn(n, generator=gen)
    say(f"[gpu] ppo head: n={n} actions={a} spread={spread}")
    clip, ent_coef, vf_coef = 0.1, 0.01, 0.5
    dev = torch.device("cuda")
    for scale in (1.0, -2.5):
        ref_l = logits.clone().requires_grad_(True)
        ref_v = value.clone().requires_grad_(True)
        want_loss, want_cf = _reference_loss(ref_l, ref_v, actions, old_logprob, advantages, returns, clip, ent_coef,
                                             vf_coef)
        (scale * want_loss).backward()
        gl = logits.to(dev).requires_grad_(True)
        gv = value.to(dev).requires_grad_(True)
        accum = torch.tensor([1.0, 2.0], device=dev)
        loss, cf = P.ppo_head_loss(gl, gv, actions.to(dev), old_logprob.to(dev), advantages.to(dev),
                                   returns.to(dev), clip, ent_coef, vf_coef, accum)
        (scale * loss).backward()
        torch.cuda.synchronize()
        torch.testing.assert_close(loss.detach().cpu(), want_loss.detach(), rtol=1e-5, atol=1e-6)
        torch.testing.assert_close(cf.cpu(), want_cf, rtol=0, atol=0.5 / n)
        torch.testing.assert_close(accum.cpu(), torch.stack([1.0 + want_loss.detach(), 2.0 + want_cf]),
                                   rtol=1e-5, atol=1e-5)
        torch.testing.assert_close(gl.grad.cpu(), ref_l.grad, rtol=1e-4, atol=1e-7)
        torch.testing.assert_close(gv.grad.cpu(), ref_v.grad, rtol=1e-4, atol=1e-7)
    if spread == 0.0:
        assert float(want_cf) == 0.0


def test_ppo_update_at_full_size_sampled():
    """One PPO update of the benchmark's configuration at full size: 8,192
    consoles x 128 steps on 8 snapshot levels with the x-delta rule and
    auto-reset, 12-way actions, Xavier init, GAE, 4 epochs of minibatch
    8,192.  Sampled consoles' rewards and dones at every rollout step equal
    oracle consoles fed the same controller masks (restoring their level's
    snapshot after each done); the update changes every parameter."""
    rom = synthrom.make_rom(2026).rom
    say("[gpu] ppo full size: snapshot bank")
    snaps = warm_snapshots(rom, [100, 180, 260, 340, 420, 500, 580, 660], seed=77)
    for i, s in enumerate(snaps):
        s[O.OFF["ram"] + synthrom.DONE_BYTE] = 3 + 2 * i        # episodes of 24-136 frames
    n, T = 8192, 128
    levels = np.random.default_rng(78).integers(0, 8, n)
    reward = dict(kind="x_delta", x_lo=synthrom.X_LO, x_hi=synthrom.X_HI, done_addr=synthrom.DONE_BYTE,
                  clip=15, time_penalty=0.01)
    cfg = P.NativePPOConfig("synthetic.nes", num_envs=n, n_steps=T, batch_size=8192, update_epochs=4,
                            frameskip=4, action_space="complex", init="xavier", reward=reward,
                            total_timesteps=n * T, save_checkpoints=False, seed=1,
                            env_to_level=tuple(int(x) for x in levels))
    rng = np.random.default_rng(2)
    sample = sorted({0, 1, 63, 64, 4095, 4096, n - 1, *rng.integers(0, n, 7).tolist()})
    rec = []
    say(f"[gpu] ppo full size: N={n} T={T} minibatch 8192 x 4 epochs, sample={sample}")
    stats = P.train_native_ppo(cfg, rom_bytes=rom, snapshot_bytes=[bytes(s) for s in snaps],
                               record=lambda k, m, r, d: rec.append((m[sample].cpu().numpy(),
                                                                     r[sample].cpu().numpy().copy(),
                                                                     d[sample].cpu().numpy().copy())))
    assert stats["updates"] == 1 and len(rec) == T
    assert math.isfinite(stats["log"][-1]["loss"])
    ob = OracleBatch(rom, list(range(len(sample))), reward=dict(kind=1, x_lo=synthrom.X_LO, x_hi=synthrom.X_HI,
                                                                done_addr=synthrom.DONE_BYTE, clip=15,
                                                                time_penalty=0.01))
    for j, c in enumerate(ob.cons):
        c.load(snaps[levels[sample[j]]])
    ends = 0
    for k, (masks, rew, done) in enumerate(rec):
        _, want_r, want_d = ob.step(masks, 4)
        np.testing.assert_array_equal(rew, want_r, err_msg=f"step {k} rewards")
        np.testing.assert_array_equal(done, want_d.astype(bool), err_msg=f"step {k} dones")
        for j in np.nonzero(want_d)[0]:
            ob.cons[j].load(snaps[levels[sample[j]]])
        ends += int(want_d.sum())
    assert ends >= len(sample)
    torch.manual_seed(cfg.seed)
    init = P._make_model(2048, 12, 256, "xavier", torch.device("cuda"))
    assert all(not torch.equal(a, b) for a, b in zip(init.parameters(), stats["model"].parameters()))
