"""nanorts_amd: the NanoRTS batched game hot path, MI355X-native.

env.step (Java admission order, durative timers, CANCEL_BOTH / RANDOM /
ALTERNATING conflict resolution), get_avail_actions legality masks, sight
radius visibility and the symbolic / pixel observation encoders run as
hand-written gfx950 HIP kernels, one wave64 per game, over thousands of games.
The Python surface mirrors the reference's JaxMARL MultiAgentEnv
(`make`, `reset`, `step`, `get_avail_actions`, `get_slot_cells`), batched over
a leading env dimension.
"""
from nanorts_amd.content import (
    CAPACITY_PROFILES,
    MAP_DIRECTORY,
    ContentError,
    GameConfig,
    UnitRecord,
    build_game,
    load_game,
    map_name_to_scenario,
    scenario_names,
    shipped_map,
    with_unit_type_table,
)
from nanorts_amd.model import ConflictStrategy, ModelError, UnitTypeTableVersion
from nanorts_amd.rendering import RenderAssets, RenderError, prepare_assets

__all__ = [
    "CAPACITY_PROFILES",
    "MAP_DIRECTORY",
    "ConflictStrategy",
    "ContentError",
    "GameConfig",
    "ModelError",
    "RenderAssets",
    "RenderError",
    "UnitRecord",
    "UnitTypeTableVersion",
    "build_game",
    "load_game",
    "make",
    "map_name_to_scenario",
    "prepare_assets",
    "scenario_names",
    "shipped_map",
    "with_unit_type_table",
]


def make(env_id: str, **kwargs):
    """nanorts.make("NanoRTS", scenario=...) (src/nanorts/adapters/jaxmarl/facade.py:43-56)."""
    from nanorts_amd.env import make as _make

    return _make(env_id, **kwargs)
