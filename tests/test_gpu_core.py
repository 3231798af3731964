"""GPU parity of the core-level functions (nanorts_amd.core) against the
oracle: reset, step with keys, legal_commands in both forms, visibility,
symbolic and pixel observations per observer, and pixels from feature maps."""
from __future__ import annotations

import sys

import numpy as np
import pytest

from tests.helpers import advanced_states, assert_states_equal, game_for

pytestmark = pytest.mark.gpu

FIELDS = ("kind", "direction", "none_duration", "target_cell", "produced_type", "request_order")


def _core_state(state_np):
    import torch

    from nanorts_amd.env import State
    from nanorts_amd.model import LEAF_NAMES

    return State({name: torch.as_tensor(np.ascontiguousarray(state_np[name]), device="cuda:0") for name in LEAF_NAMES})


@pytest.mark.parametrize("case", ["16x16-random-partial", "barracks-random", "gow-alternating"])
def test_core_functions_match_oracle(case, oracle_threads):
    import torch

    from nanorts_amd import core, rendering

    print(f"core functions {case}", flush=True)
    sys.stdout.flush()
    torch.cuda.set_device(0)
    game, partial = game_for(case)
    L = 8 if case.startswith("gow") else 48
    oracle, st = advanced_states(game, L, 60 if case.startswith("gow") else 150, partial, oracle_threads, seed=71)
    fresh = core.reset((0, 1), game, 3, device="cuda:0")
    for name, value in game.initial_state.items():
        np.testing.assert_array_equal(fresh.leaves[name].cpu().numpy()[1], value, err_msg=name)
    state = _core_state(st)
    rows = core.legal_commands(state, game).cpu().numpy()
    np.testing.assert_array_equal(rows, oracle.legality_rows(st))
    words = core.legal_commands(state, game, stored="words").cpu().numpy().view(np.uint32)
    bits = np.unpackbits(words.view(np.uint8), bitorder="little").reshape(*words.shape[:-1], 96)[..., :rows.shape[-1]]
    np.testing.assert_array_equal(bits.astype(bool), rows)
    for observer in (0, 1):
        np.testing.assert_array_equal(core.visibility(game, state, observer=observer).cpu().numpy(),
                                      oracle.visible_cells(st, observer))
        maps, scalars = oracle.symbolic(st, partial)
        got = core.symbolic(game, state, observer=observer, partial_observability=partial)
        np.testing.assert_array_equal(got.feature_maps.cpu().numpy(), maps[:, observer])
        np.testing.assert_array_equal(got.scalars.cpu().numpy(), scalars[:, observer])
    if not case.startswith("gow"):
        assets = rendering.prepare_assets(game.bucket)
        image, _ = oracle.pixels(st, partial, assets.tiles)
        got = core.pixels(game, state, assets, observer=1, partial_observability=partial)
        np.testing.assert_array_equal(got.image.cpu().numpy(), image[:, 1])
        full, _ = oracle.symbolic(st, False)
        want_full, _ = oracle.pixels(st, False, assets.tiles)
        drawn = core.pixels_from_symbolic(torch.as_tensor(full, device="cuda:0"), assets, game)
        np.testing.assert_array_equal(drawn.cpu().numpy(), want_full)
    rng = np.random.default_rng(5)
    keys = rng.integers(0, 2**32, size=(L, 2), dtype=np.uint64).astype(np.uint32)
    cmds = oracle.decode_actions(st, oracle.sample_actions(oracle.avail_rows(st), (2, 3), 1))
    out = core.step(keys, state, {f: torch.as_tensor(cmds[f], device="cuda:0") for f in FIELDS}, game)
    want = oracle.core_step(st, cmds, keys)
    got = {name: t.cpu().numpy() for name, t in state.leaves.items()}
    assert_states_equal(st, {**got, "environment_root": st["environment_root"], "episode_index": st["episode_index"]},
                        "core.step")
    np.testing.assert_array_equal(out["reward"].cpu().numpy(), want["reward"])
    np.testing.assert_array_equal(out["admitted_produce"].cpu().numpy(), want["admitted_produce"])
