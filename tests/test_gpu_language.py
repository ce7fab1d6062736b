"""Language semantics of the newt DSL on the GPU (HIP backend), following the
behaviours the reference's test suite pins (tests/test_ops.py,
tests/test_control_flow.py, tests/test_review_fixes.py)."""

import numpy as np
import pytest
import torch

import newt_amd as newt
import newt_amd.language as nl

pytestmark = pytest.mark.gpu


@newt.jit
def _grid_ids(out_ptr):
    x = nl.program_id(0)
    y = nl.program_id(1)
    z = nl.program_id(2)
    nx = nl.num_programs(0)
    ny = nl.num_programs(1)
    lin = x + nx * (y + ny * z)
    nl.store(out_ptr + lin * 3, x)
    nl.store(out_ptr + lin * 3 + 1, y)
    nl.store(out_ptr + lin * 3 + 2, z)


@pytest.mark.parametrize("grid", [(7,), (8,), (37, 3), (16, 16), (5, 3, 7), (1, 1, 1), (1000,)])
def test_program_ids_cover_grid_once(grid):
    """Every program id tuple of the grid runs exactly once (the backend
    renumbers workgroups across XCDs; the renumbering must be a bijection)."""
    g = tuple(grid) + (1,) * (3 - len(grid))
    n = g[0] * g[1] * g[2]
    out = torch.full((n * 3,), -1, dtype=torch.int32, device="cuda")
    _grid_ids[grid](out)
    torch.cuda.synchronize()
    ids = out.view(n, 3).cpu().numpy()
    lin = np.arange(n)
    want = np.stack([lin % g[0], (lin // g[0]) % g[1], lin // (g[0] * g[1])], axis=1)
    assert np.array_equal(ids, want)
