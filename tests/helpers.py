"""Shared test helpers: game cases, oracle-generated states, host/device moves."""
from __future__ import annotations

import numpy as np

from nanorts_amd.content import map_name_to_scenario
from nanorts_amd.model import ConflictStrategy, UnitTypeTableVersion
from oracle.oracle import Oracle, batch_initial, copy_state

# (name, map, utt, strategy, max_cycles, capacity_profile, partial)
CASES = {
    "8x8-original-both": ("basesWorkers8x8", UnitTypeTableVersion.ORIGINAL, ConflictStrategy.CANCEL_BOTH, 5000, True,
                          False),
    "16x16-finetuned-both": ("basesWorkers16x16", UnitTypeTableVersion.ORIGINAL_FINETUNED,
                             ConflictStrategy.CANCEL_BOTH, 5000, True, False),
    "16x16-random-partial": ("basesWorkers16x16", UnitTypeTableVersion.ORIGINAL_FINETUNED,
                             ConflictStrategy.CANCEL_RANDOM, 5000, True, True),
    "16x16-alternating": ("basesWorkers16x16", UnitTypeTableVersion.ORIGINAL_FINETUNED,
                          ConflictStrategy.CANCEL_ALTERNATING, 300, True, False),
    "16x16-noprofile-random": ("basesWorkers16x16", UnitTypeTableVersion.ORIGINAL, ConflictStrategy.CANCEL_RANDOM,
                               5000, False, True),
    "gow-alternating": ("GardenOfWar64x64", UnitTypeTableVersion.ORIGINAL_FINETUNED,
                        ConflictStrategy.CANCEL_ALTERNATING, 5000, False, False),
    "melee-both": ("melee8x8Mixed4", UnitTypeTableVersion.ORIGINAL_FINETUNED, ConflictStrategy.CANCEL_BOTH, 200, True,
                   True),
    "barracks-random": ("basesWorkersBarracks8x8", UnitTypeTableVersion.ORIGINAL, ConflictStrategy.CANCEL_RANDOM, 150,
                        True, True),
    "obstacle-alternating": ("basesWorkers8x8Obstacle", UnitTypeTableVersion.ORIGINAL,
                             ConflictStrategy.CANCEL_ALTERNATING, 120, True, False),
    # Ranged units (attack range 3) from the first cycle: the samplers' general
    # attack window next to the range-1 neighbour masks
    "ranged-random": ("melee8x8Mixed6", UnitTypeTableVersion.ORIGINAL_FINETUNED, ConflictStrategy.CANCEL_RANDOM, 300,
                      True, True),
    # widths that are not a multiple of 4: the kernels' general observation
    # and summary branches
    "10x10-random-partial": ("basesWorkers10x10", UnitTypeTableVersion.ORIGINAL_FINETUNED,
                             ConflictStrategy.CANCEL_RANDOM, 5000, True, True),
    "9x8-alternating": ("NoWhereToRun9x8", UnitTypeTableVersion.ORIGINAL, ConflictStrategy.CANCEL_ALTERNATING, 130,
                        True, False),
    # boards 17-32 wide: the 32-bit row masks of the visibility and window
    # passes, with walls (barricades) and partial observability
    "24x24-barricades-alternating": ("barricades24x24", UnitTypeTableVersion.ORIGINAL_FINETUNED,
                                     ConflictStrategy.CANCEL_ALTERNATING, 5000, True, True),
    "32x32-random-partial": ("basesWorkers32x32A", UnitTypeTableVersion.ORIGINAL_FINETUNED,
                             ConflictStrategy.CANCEL_RANDOM, 5000, True, True),
}


def game_for(case: str):
    name, utt, strategy, max_cycles, profile, partial = CASES[case]
    game = map_name_to_scenario(name, utt=utt, conflict_strategy=strategy, max_cycles=max_cycles,
                                capacity_profile=profile)
    return game, partial


def roots(num_envs: int, salt: int = 0) -> np.ndarray:
    i = np.arange(num_envs, dtype=np.uint32)
    return np.stack([i * np.uint32(2654435761) + np.uint32(salt), i ^ np.uint32(0x9E3779B9 + salt)], 1).astype(np.uint32)


def advanced_states(game, num_envs: int, steps: int, partial: bool, threads: int, seed: int = 7):
    """Mid-game states: `steps` oracle rollout cycles from the initial state."""
    oracle = Oracle(game)
    state = batch_initial(game, num_envs, roots(num_envs, seed))
    if steps:
        oracle.rollout(state, (seed, seed + 1), 0, steps, partial, threads=threads, record=False)
    return oracle, state


def to_device(env, state_np):
    import torch

    from nanorts_amd.env import EnvironmentState, State
    from nanorts_amd.model import LEAF_NAMES

    d = env.device
    leaves = {name: torch.as_tensor(np.ascontiguousarray(state_np[name]), device=d) for name in LEAF_NAMES}
    return EnvironmentState(State(leaves),
                            torch.as_tensor(np.ascontiguousarray(state_np["environment_root"]).view(np.int32), device=d),
                            torch.as_tensor(np.ascontiguousarray(state_np["episode_index"]).view(np.int32), device=d))


def to_host(env_state) -> dict[str, np.ndarray]:
    out = {name: t.cpu().numpy() for name, t in env_state.core_state.leaves.items()}
    out["environment_root"] = env_state.environment_root.cpu().numpy().view(np.uint32)
    out["episode_index"] = env_state.episode_index.cpu().numpy().view(np.uint32)
    return out


def assert_states_equal(expected: dict[str, np.ndarray], actual: dict[str, np.ndarray], where: str = "") -> None:
    for name, want in expected.items():
        got = actual[name]
        w = np.asarray(want)
        g = np.asarray(got).astype(w.dtype) if w.dtype == np.bool_ else np.asarray(got)
        if not np.array_equal(w.astype(np.int64) if w.dtype != np.bool_ else w,
                              g.astype(np.int64) if g.dtype != np.bool_ else g):
            bad = np.argwhere((w != g).reshape(w.shape[0], -1).any(1)).ravel()
            raise AssertionError(f"{where}: leaf {name} differs in envs {bad[:10].tolist()} "
                                 f"(first env: want {w[bad[0]].ravel()[:24]}, got {g[bad[0]].ravel()[:24]})")


__all__ = ["CASES", "game_for", "roots", "advanced_states", "to_device", "to_host", "assert_states_equal",
           "copy_state"]
