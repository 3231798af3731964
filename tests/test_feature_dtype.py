"""Feature-map dtype selection of the symbolic surface (CPU only): the
narrowest published dtype that holds the content's bounds
(src/nanorts/adapters/jaxmarl/layout.py:146-158,
src/nanorts/observations/symbolic.py:183-220), explicit wider dtypes, and
the refusal of content whose values a byte cannot hold."""
from __future__ import annotations

import numpy as np
import pytest
import torch

from nanorts_amd.content import UnitRecord, build_game, map_name_to_scenario
from nanorts_amd.env import feature_bounds, feature_dtype, feature_dtype_for_surface
from nanorts_amd.model import ModelError


def _game(pile: int):
    units = [UnitRecord("Resource", 1, -1, 0, 0, 1, pile), UnitRecord("Base", 2, 0, 1, 1, 10, 0),
             UnitRecord("Worker", 3, 0, 2, 1, 1, 0), UnitRecord("Base", 4, 1, 3, 3, 10, 0),
             UnitRecord("Worker", 5, 1, 2, 3, 1, 0)]
    return build_game(width=4, height=4, terrain="0" * 16, players=[5, 5], units=units)


def test_bounds_of_shipped_content():
    """basesWorkers16x16 (FINETUNED): Heavy has 8 hit points, the piles hold 25."""
    bounds = feature_bounds(map_name_to_scenario("basesWorkers16x16"))
    assert bounds == {"hit_points": 10, "carried_resources": 25, "owner": 2, "unit_type": 7,
                      "pending_action_kind": 5, "terrain": 1}


def test_narrowest_dtype_is_uint8_for_every_byte_sized_content():
    assert feature_dtype(map_name_to_scenario("basesWorkers16x16")) == torch.uint8
    assert feature_dtype(_game(255)) == torch.uint8


@pytest.mark.parametrize("requested,want", [("uint8", torch.uint8), (np.int16, torch.int16),
                                            (torch.int32, torch.int32), ("int32", torch.int32)])
def test_explicit_dtypes(requested, want):
    assert feature_dtype(_game(20), requested) == want


def test_refusals():
    with pytest.raises(ModelError, match="not one of"):
        feature_dtype(_game(20), "float32")
    with pytest.raises(ModelError, match="cannot hold"):  # a pile of 300 does not fit uint8
        feature_dtype(_game(300), "uint8")
    # the narrowest holding dtype would be int16, but the kernels encode bytes
    with pytest.raises(ModelError, match="one byte per feature"):
        feature_dtype(_game(300))
    with pytest.raises(ModelError, match="one byte per feature"):
        feature_dtype(_game(300), "int32")
    # the pixel surface publishes no feature maps but draws from the bytes
    with pytest.raises(ModelError, match="one byte per feature"):
        feature_dtype_for_surface(_game(300), "pixels", None)
    assert feature_dtype_for_surface(_game(20), "pixels", None) == torch.uint8
