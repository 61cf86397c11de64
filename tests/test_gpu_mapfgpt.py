"""GPU parity of the MAPF-GPT builder (jl_mapfgpt_*) against the C oracle.

Ports /root/reference/tests/expert/test_mapf_gpt_cuda.py to the gfx950 path
and adds oracle parity on maze maps (C3 shape).  Bit-exact: tokens, labels,
active mask, cost-to-go fields, histories, diagnostics.
"""
import numpy as np
import pytest

torch = pytest.importorskip("torch")
pytestmark = pytest.mark.gpu


def ext128():
    from iclr_2027_jointoom_amd import profile

    return profile(128, 128)


def _grids(ext, num_envs=2, *, device="cuda", dtype=torch.int32):
    return torch.zeros((num_envs, ext.COMPILED_MAP_W, ext.COMPILED_MAP_H), dtype=dtype, device=device)


def _valid_rows(num_envs=2, num_agents=4):
    rows = torch.zeros((num_envs * num_agents, 13), dtype=torch.int16, device="cuda")
    blocks = rows.view(num_envs, num_agents, 13)
    blocks[:, :, 0] = torch.arange(num_envs, dtype=torch.int16, device="cuda")[:, None]
    blocks[:, :, 1] = torch.arange(num_agents, dtype=torch.int16, device="cuda")[None, :]
    blocks[:, :, 2] = 10
    blocks[:, :, 3] = torch.arange(num_agents, dtype=torch.int16, device="cuda")[None, :] + 10
    blocks[:, :, 4] = 20
    blocks[:, :, 5] = torch.arange(num_agents, dtype=torch.int16, device="cuda")[None, :] + 10
    blocks[:, :, 7] = 1
    blocks[:, :, 8:13] = 5
    return rows


def test_api_shapes_and_no_pyg_attributes():
    ext = ext128()
    b = ext.MapfGPTObservationBuilder(_grids(ext), 4)
    assert b.tokens.shape == (8, 256) and b.tokens.dtype == torch.int32
    assert b.labels.shape == (8,) and b.labels.dtype == torch.int64
    assert b.cost_to_go.shape == (2, 4, 128, 128) and b.cost_to_go.dtype == torch.int16
    assert b.state_packed.shape == (8, 8) and b.state_packed.dtype == torch.int16
    assert b.agent_at_cell.shape == (2, 128, 128) and b.agent_at_cell.dtype == torch.int32
    assert b.pyg_ptr.tolist() == [0, 4, 8]
    for name in ("pyg_edge_index_storage", "pyg_edge_attr_storage", "pyg_x"):
        assert not hasattr(b, name)


def test_memory_inventory_without_allocation():
    ext = ext128()
    b = ext.MapfGPTObservationBuilder(_grids(ext), 4)
    torch.cuda.synchronize()
    before = torch.cuda.memory_allocated()
    inv = b.memory_tensors
    torch.cuda.synchronize()
    assert torch.cuda.memory_allocated() == before
    assert inv["goal_cache"].shape == (8, 2) and inv["tokens"] is b.tokens


def test_active_mask():
    ext = ext128()
    b = ext.MapfGPTObservationBuilder(_grids(ext, 1), 4)
    rows = _valid_rows(1, 4)
    rows[0, 4:6] = rows[0, 2:4]
    rows[2, 4:6] = rows[2, 2:4]
    b.build_tokens(rows)
    assert b.active_mask.dtype == torch.bool and b.active_mask.cpu().tolist() == [False, True, False, True]


def test_work_is_owned_by_current_stream():
    ext = ext128()
    A = 512
    b = ext.MapfGPTObservationBuilder(_grids(ext, 1), A)
    src = _valid_rows(1, A)
    ids = torch.arange(A, dtype=torch.int16, device="cuda")
    src[:, 2] = ids // 64 + 20
    src[:, 3] = ids % 64 + 20
    src[:, 4] = 100
    src[:, 5] = src[:, 3]
    src[:, 6] = ids % 5
    delayed = torch.zeros_like(src)
    stream = torch.cuda.Stream()
    done = torch.cuda.Event()
    default_done = torch.cuda.Event()
    torch.cuda.synchronize()
    with torch.cuda.stream(stream):
        torch.cuda._sleep(50_000_000)
        delayed.copy_(src)
        b.build_tokens(delayed)
        done.record()
    default_done.record(torch.cuda.default_stream())
    done.synchronize()
    assert default_done.query(), "builder work escaped to the default stream"
    assert b.labels.cpu().tolist() == (ids % 5).cpu().tolist()
    assert b.diagnostics.cpu().tolist() == [0, 0, 0, 0]


@pytest.mark.parametrize("grids, message", [
    (lambda e: _grids(e, device="cpu"), "CUDA"),
    (lambda e: _grids(e, dtype=torch.float32), "int32"),
    (lambda e: torch.zeros((1, 8, 8), dtype=torch.int32, device="cuda"), "shape"),
])
def test_rejects_invalid_grids(grids, message):
    ext = ext128()
    with pytest.raises(RuntimeError, match=message):
        ext.MapfGPTObservationBuilder(grids(ext), 4)


def test_rejects_invalid_layouts():
    ext = ext128()
    b = ext.MapfGPTObservationBuilder(_grids(ext), 4)
    rows = _valid_rows()
    with pytest.raises(RuntimeError, match="int16"):
        b.build_tokens(rows.to(torch.int32))
    with pytest.raises(RuntimeError, match="13"):
        b.build_tokens(rows[:, :8].contiguous())
    with pytest.raises(RuntimeError, match="row count"):
        b.build_tokens(rows[:-1].contiguous())
    backing = torch.empty((8, 26), dtype=torch.int16, device="cuda")
    nc = backing[:, ::2]
    nc.copy_(rows)
    with pytest.raises(RuntimeError, match="contiguous"):
        b.build_tokens(nc)
    b2 = ext.MapfGPTObservationBuilder(_grids(ext, 1), 2)
    valid = torch.tensor([[10, 11]], dtype=torch.int16, device="cuda")
    with pytest.raises(RuntimeError, match="int16"):
        b2.build_tokens_from_state(valid.to(torch.int32), valid, valid, valid)
    with pytest.raises(RuntimeError, match="shape"):
        b2.build_tokens_from_state(valid[:, :1].contiguous(), valid, valid, valid)
    with pytest.raises(RuntimeError, match="uint8"):
        b2.append_actions(valid)
    with pytest.raises(RuntimeError, match="shape"):
        b2.append_actions(torch.zeros((1, 1), dtype=torch.uint8, device="cuda"))
    # the wrappers' one-test fast path falls back to the detailed messages
    wide = torch.tensor([[10, 0, 11, 0]], dtype=torch.int16, device="cuda")
    with pytest.raises(RuntimeError, match="cur_y must be contiguous"):
        b2.build_tokens_from_state(valid, wide[:, ::2], valid, valid)
    with pytest.raises(RuntimeError, match="goal_x must be on a CUDA device"):
        b2.build_tokens_from_state(valid, valid, valid.cpu(), valid)
    acts = torch.zeros((1, 4), dtype=torch.uint8, device="cuda")
    with pytest.raises(RuntimeError, match="actions must be contiguous"):
        b2.append_actions(acts[:, ::2])
    with pytest.raises(RuntimeError, match="actions must be on a CUDA device"):
        b2.append_actions(acts[:, :2].cpu())
    b2.build_tokens_from_state(valid, valid, valid, valid)  # valid tensors still pass
    b2.append_actions(acts[:, :2].contiguous())


def test_invalid_position_is_diagnosed():
    ext = ext128()
    b = ext.MapfGPTObservationBuilder(_grids(ext, 1), 1)
    rows = _valid_rows(1, 1)
    rows[0, 2] = 128
    b.build_tokens(rows)
    assert b.diagnostics.cpu().tolist()[3] > 0
    assert bool((b.tokens == 66).all())


def _unsigned(b):
    return b.cost_to_go.to(torch.int32).bitwise_and(0xFFFF)


def test_cost_to_go_exact_uint16_beyond_254():
    ext = ext128()
    grid = torch.ones((1, 128, 128), dtype=torch.int32, device="cuda")
    grid[0, 0, :] = 0
    grid[0, 1, -1] = 0
    grid[0, 2, :] = 0
    b = ext.MapfGPTObservationBuilder(grid, 1)
    rows = _valid_rows(1, 1)
    rows[0, 2:6] = torch.tensor([2, 0, 0, 0], dtype=torch.int16, device="cuda")
    rows[0, 7] = 0
    b.build_tokens(rows)
    cost = _unsigned(b)[0, 0]
    assert cost[0, 0].item() == 0 and cost[0, 1].item() == 1
    assert cost[2, 0].item() == 256 and cost[3, 0].item() == 65535
    assert b.diagnostics[0].item() == 0


def test_goal_change_refresh_and_replay():
    ext = ext128()
    b = ext.MapfGPTObservationBuilder(_grids(ext, 1), 1)
    ra = _valid_rows(1, 1)
    ra[0, 2:6] = torch.tensor([10, 10, 10, 20], dtype=torch.int16, device="cuda")
    ra[0, 7] = 0
    rb = ra.clone()
    rb[0, 4:6] = torch.tensor([30, 30], dtype=torch.int16, device="cuda")
    b.build_tokens(ra)
    ca = _unsigned(b).clone()
    b.build_tokens(rb)
    cb = _unsigned(b).clone()
    b.build_tokens(ra)
    assert ca[0, 0, 10, 20].item() == 0 and cb[0, 0, 30, 30].item() == 0
    assert not torch.equal(ca, cb) and torch.equal(ca, _unsigned(b))


def _parity_fixture(num_agents=16):
    grid = np.zeros((128, 128), dtype=np.int32)
    grid[7:25, 17] = 1
    grid[15, 17] = 0
    positions = [(15, 15)]
    for dx in range(-2, 3):
        for dy in range(-2, 3):
            if len(positions) >= num_agents:
                break
            pos = (15 + dx, 15 + dy)
            if pos != positions[0] and grid[pos] == 0:
                positions.append(pos)
    rows = np.zeros((num_agents, 13), dtype=np.uint16)
    rows[:, 1] = np.arange(num_agents)
    rows[:, 2:4] = positions[:num_agents]
    rows[:, 4] = 25
    rows[:, 5] = np.arange(num_agents) % 10 + 20
    rows[:, 6] = np.arange(num_agents) % 5
    rows[:, 7] = 1
    for a in range(num_agents):
        rows[a, 8:13] = [5 if s < 2 else (a + s) % 5 for s in range(5)]
    return grid[None], rows


def test_parity_fixture_matches_oracle(oracle):
    grids, rows = _parity_fixture()
    ob = oracle.OracleMapfGPT(grids, 16)
    ob.build_rows(rows)
    ext = ext128()
    b = ext.MapfGPTObservationBuilder(torch.from_numpy(grids).cuda(), 16)
    b.build_tokens(torch.from_numpy(rows.astype(np.int16)).cuda())
    assert np.array_equal(b.tokens.cpu().numpy(), ob.tokens)
    assert np.array_equal(b.labels.cpu().numpy(), ob.labels)
    assert np.array_equal(b.cost_to_go.cpu().numpy(), ob.cost_to_go.view(np.int16))
    assert b.diagnostics.cpu().tolist() == [0, 0, 0, 0]
    # agent_at_cell on request equals the oracle's scatter
    assert np.array_equal(b.agent_at_cell.cpu().numpy(), ob.agent_at_cell)


def test_replay_determinism_and_resident_equals_raw():
    grids, rows_a = _parity_fixture()
    rows_b = rows_a.copy()
    rows_b[:, 4] = 30
    ext = ext128()
    g = torch.from_numpy(grids).cuda()
    b = ext.MapfGPTObservationBuilder(g, 16)
    ra = torch.from_numpy(rows_a.astype(np.int16)).cuda()
    rb = torch.from_numpy(rows_b.astype(np.int16)).cuda()
    b.build_tokens(ra)
    ta = b.tokens.clone()
    b.build_tokens(rb)
    b.build_tokens(ra)
    assert torch.equal(ta, b.tokens)
    grids8, rows8 = _parity_fixture(8)
    g8 = torch.from_numpy(grids8).cuda()
    r8 = torch.from_numpy(rows8.astype(np.int16)).cuda()
    raw = ext.MapfGPTObservationBuilder(g8, 8)
    res = ext.MapfGPTObservationBuilder(g8, 8)
    res.histories.copy_(r8[:, 8:13])
    raw.build_tokens(r8)
    blk = r8.view(1, 8, 13)
    res.build_tokens_from_state(blk[:, :, 2].contiguous(), blk[:, :, 3].contiguous(),
                                blk[:, :, 4].contiguous(), blk[:, :, 5].contiguous())
    assert torch.equal(res.tokens, raw.tokens) and torch.equal(res.active_mask, raw.active_mask)
    assert res.diagnostics.cpu().tolist() == [0, 0, 0, 0]


def test_history_roll_kat():
    ext = ext128()
    b = ext.MapfGPTObservationBuilder(_grids(ext, 1), 3)
    cx = torch.tensor([[10, 11, 12]], dtype=torch.int16, device="cuda")
    gx = torch.tensor([[20, 11, 22]], dtype=torch.int16, device="cuda")
    b.reset_histories()
    b.build_tokens_from_state(cx, cx, gx, gx)
    assert b.histories.cpu().tolist() == [[5] * 5] * 3
    assert b.active_mask.cpu().tolist() == [True, False, True]
    b.append_actions(torch.tensor([[1, 4, 3]], dtype=torch.uint8, device="cuda"))
    assert b.histories.cpu().tolist() == [[5, 5, 5, 5, 1], [5, 5, 5, 5, 0], [5, 5, 5, 5, 3]]
    b.build_tokens_from_state(cx, cx, gx, gx)
    rows = torch.zeros((3, 13), dtype=torch.int16, device="cuda")
    rows[:, 1] = torch.arange(3, dtype=torch.int16, device="cuda")
    rows[:, 2] = cx[0]
    rows[:, 3] = cx[0]
    rows[:, 4] = gx[0]
    rows[:, 5] = gx[0]
    rows[:, 8:13] = b.histories
    ref = ext.MapfGPTObservationBuilder(_grids(ext, 1), 3)
    ref.build_tokens(rows)
    assert torch.equal(b.tokens, ref.tokens)
    # out-of-range action: counted in diagnostics[1], recorded as 0
    b.append_actions(torch.tensor([[7, 0, 0]], dtype=torch.uint8, device="cuda"))
    assert b.diagnostics.cpu().tolist()[1] == 1 and b.histories[0, 4].item() == 0


@pytest.mark.parametrize("E,A", [(2, 256), (3, 100), (1, 7)])
def test_append_actions_histories_match_oracle(oracle, E, A):
    """Full 256-agent segments move as 16-byte words, a partial last segment
    element by element; out-of-range actions count in diagnostics[1]."""
    from iclr_2027_jointoom_amd import profile
    from iclr_2027_jointoom_amd.synthetic import make_batch

    grids, starts, goals = make_batch(11, E, 32, 32, A)
    b = profile(32, 32).MapfGPTObservationBuilder(torch.from_numpy(grids.astype(np.int32)).cuda(), A)
    ob = oracle.OracleMapfGPT(grids, A)
    cx, cy = starts[..., 0].copy(), starts[..., 1].copy()
    gx, gy = goals[..., 0].copy(), goals[..., 1].copy()
    rng = np.random.default_rng(E * 1000 + A)
    rejected = 0
    for it in range(4):
        b.build_tokens_from_state(*(torch.from_numpy(v).cuda() for v in (cx, cy, gx, gy)))
        ob.build_state(cx, cy, gx, gy)
        acts = rng.integers(0, 7, size=(E, A), dtype=np.uint8)  # 5 and 6 are rejected
        b.append_actions(torch.from_numpy(acts).cuda())
        ob.append(acts)
        torch.cuda.synchronize()
        assert np.array_equal(b.histories.cpu().numpy().view(np.uint16), ob.histories), it
        assert b.diagnostics.cpu().tolist() == ob.diagnostics.tolist(), it
        rejected += int(ob.diagnostics[1])
    assert rejected > 0


@pytest.mark.parametrize("num_agents", [256, 512])
def test_scales_beyond_visible_cap(num_agents):
    ext = ext128()
    rows = _valid_rows(1, num_agents)
    ids = torch.arange(num_agents, dtype=torch.int16, device="cuda")
    rows[:, 2] = ids // 64 + 20
    rows[:, 3] = ids % 64 + 20
    rows[:, 4] = 100
    rows[:, 5] = ids % 64 + 20
    b = ext.MapfGPTObservationBuilder(_grids(ext, 1), num_agents)
    b.build_tokens(rows)
    assert b.tokens.shape == (num_agents, 256)
    assert bool(((b.tokens >= 0) & (b.tokens <= 66)).all()) and b.diagnostics[0].item() == 0


@pytest.mark.parametrize("kind,E,W,A", [("maze", 64, 64, 128), ("iid", 32, 32, 64), ("iid", 4, 128, 512)])
def test_maze_batches_match_oracle(oracle, kind, E, W, A):
    """C3 shape on fewer envs: BFS fields + tokens of fresh goals, then a
    steady-state rebuild with moved agents and appended histories."""
    from iclr_2027_jointoom_amd import profile
    from iclr_2027_jointoom_amd.synthetic import make_batch

    grids, starts, goals = make_batch(7 + W, E, W, W, A, kind=kind)
    ext = profile(W, W)
    g = torch.from_numpy(grids.astype(np.int32)).cuda()
    b = ext.MapfGPTObservationBuilder(g, A)
    ob = oracle.OracleMapfGPT(grids, A)
    cx, cy = starts[..., 0].copy(), starts[..., 1].copy()
    gx, gy = goals[..., 0].copy(), goals[..., 1].copy()
    rng = np.random.default_rng(0)
    for it in range(3):
        b.build_tokens_from_state(*(torch.from_numpy(v).cuda() for v in (cx, cy, gx, gy)))
        ob.build_state(cx, cy, gx, gy)
        torch.cuda.synchronize()
        assert np.array_equal(b.cost_to_go.cpu().numpy(), ob.cost_to_go.view(np.int16)), it
        assert np.array_equal(b.tokens.cpu().numpy(), ob.tokens), it
        assert np.array_equal(b.state_packed.cpu().numpy(), ob.state_packed.view(np.int16)), it
        assert b.diagnostics.cpu().tolist() == ob.diagnostics.tolist() == [0, 0, 0, 0]
        acts = rng.integers(0, 5, size=(E, A), dtype=np.uint8)
        b.append_actions(torch.from_numpy(acts).cuda())
        ob.append(acts)
        # swap a few goals between agents of env 0 to force partial refreshes
        gx[0, :4], gy[0, :4] = gx[0, :4][::-1].copy(), gy[0, :4][::-1].copy()
        cx, cy = np.roll(cx, 1, axis=1), np.roll(cy, 1, axis=1)


def _state_parity(oracle, grids, starts, goals, A, builds=2, seed=0):
    from iclr_2027_jointoom_amd import profile

    E, W, H = grids.shape
    ext = profile(W, H)
    b = ext.MapfGPTObservationBuilder(torch.from_numpy(grids.astype(np.int32)).cuda(), A)
    ob = oracle.OracleMapfGPT(grids, A)
    cx, cy = starts[..., 0].copy(), starts[..., 1].copy()
    gx, gy = goals[..., 0].copy(), goals[..., 1].copy()
    rng = np.random.default_rng(seed)
    for it in range(builds):
        b.build_tokens_from_state(*(torch.from_numpy(v).cuda() for v in (cx, cy, gx, gy)))
        ob.build_state(cx, cy, gx, gy)
        torch.cuda.synchronize()
        assert np.array_equal(b.tokens.cpu().numpy(), ob.tokens), it
        assert np.array_equal(b.active_mask.cpu().numpy().astype(np.uint8), ob.active_mask), it
        assert b.diagnostics.cpu().tolist() == ob.diagnostics.tolist(), it
        acts = rng.integers(0, 5, size=(E, A), dtype=np.uint8)
        b.append_actions(torch.from_numpy(acts).cuda())
        ob.append(acts)
        cx, cy = np.roll(cx, 1, axis=1), np.roll(cy, 1, axis=1)
    return b, ob


def test_more_than_13_visible_agents_match_oracle(oracle):
    """Half of a 32x32 map occupied: windows hold up to ~60 agents, so the
    top-13 selection by (Manhattan, id) is exercised well past the cap."""
    from iclr_2027_jointoom_amd.synthetic import make_batch

    grids, starts, goals = make_batch(3, 2, 32, 32, 400, density=0.1)
    b, _ = _state_parity(oracle, grids, starts, goals, 400)
    # the visible-agent block is full for most egos
    full = (b.tokens[:, 121 + 12 * 10].cpu().numpy() != 66).mean()
    assert full > 0.5


def test_sparse_cell_map_on_256_maps_matches_oracle(oracle):
    """256x256 maps use the sparse cell -> agent map instead of the dense one."""
    from iclr_2027_jointoom_amd.synthetic import make_batch

    grids, starts, goals = make_batch(11, 2, 256, 256, 192)
    _state_parity(oracle, grids, starts, goals, 192)


@pytest.mark.parametrize("W,H,A", [(256, 256, 300), (100, 256, 1024), (256, 128, 520)])
def test_sparse_cell_map_with_shared_cells_matches_oracle(oracle, W, H, A):
    """Maps of more than 16,384 cells take the sparse cell -> agent map
    (occupancy bitmap, occupied cells before each word, ids in cell order):
    shared cells (two agents, four agents, ids in either order), rejected
    rows and positions off the map give the oracle's tokens and diagnostics,
    with fewer occupancy words than threads (100 x 256) and an env spread
    over two workgroups (520 agents)."""
    from iclr_2027_jointoom_amd import profile

    rng = np.random.default_rng(W * 7 + H + A)
    E = 2
    grids = (rng.random((E, W, H)) < 0.25).astype(np.int32)
    ext = profile(W, H)
    b = ext.MapfGPTObservationBuilder(torch.from_numpy(grids).cuda(), A)
    assert not b.single_launch
    ob = oracle.OracleMapfGPT(grids, A)
    rows = _rows_case(rng, grids, A)
    goals = rows[:, 4:6].copy()
    for it in range(3):
        rows = _rows_case(rng, grids, A, goals)
        rows[:, 7] = 1 if it == 0 else 0
        rows[7, 2:4] = rows[8, 2:4]                  # two agents on one cell
        rows[A + 20:A + 23, 2:4] = rows[A + 30, 2:4]  # four agents on one cell, the lowest id not first
        rows[A - 1, 2:4] = rows[0, 2:4]              # the highest id on the lowest one's cell
        if it >= 1:
            rows[5, 0] = E + 1                       # rejected row (env out of range)
            rows[A + 2, 2] = W + 3                   # position off the map
        t = torch.from_numpy(rows.astype(np.int16)).cuda()
        b.build_tokens(t)
        ob.build_rows(rows)
        torch.cuda.synchronize()
        assert np.array_equal(b.tokens.cpu().numpy(), ob.tokens), it
        assert b.diagnostics.cpu().tolist() == ob.diagnostics.tolist(), it
        assert ob.diagnostics[2] >= 5, it  # the shared cells were counted


@pytest.mark.parametrize("W,H", [(256, 256), (128, 128), (200, 96)])
def test_token_pass_windows_at_corners_and_edges_match_oracle(oracle, W, H):
    """Agents packed into the four corners and along the four edges of the
    map, so that windows reach into the empty border of the cell -> agent
    map (sparse beyond 16,384 cells, dense below) and the unreachable border
    of the tiled fields on every side; goals in the opposite corners.  The
    two-launch token pass equals the oracle over two builds."""
    from iclr_2027_jointoom_amd import profile

    E = 2
    cells = []
    for cx, cy in ((0, 0), (0, H - 1), (W - 1, 0), (W - 1, H - 1)):
        for dx in range(4):
            for dy in range(4):
                cells.append((abs(cx - dx), abs(cy - dy)))
    for k in range(6, W - 6, max(1, W // 9)):
        cells += [(k, 0), (k, H - 1)]
    for k in range(6, H - 6, max(1, H // 9)):
        cells += [(0, k), (W - 1, k)]
    cells = list(dict.fromkeys(cells))
    A = len(cells)
    grids = np.zeros((E, W, H), np.int32)
    grids[:, W // 2, 1:H - 1] = 1  # a wall through the middle with gaps at both ends
    ext = profile(W, H)
    b = ext.MapfGPTObservationBuilder(torch.from_numpy(grids).cuda(), A)
    assert not b.single_launch
    ob = oracle.OracleMapfGPT(grids.astype(np.uint8), A)
    pos = np.array(cells, np.int16)
    goal = np.stack([W - 1 - pos[:, 0], H - 1 - pos[:, 1]], -1).astype(np.int16)
    rng = np.random.default_rng(W + H)
    for it in range(2):
        p = np.stack([pos] * E)
        if it:
            p[1] = p[1][rng.permutation(A)]  # the same cells, other agents on them
        g = np.stack([goal] * E)
        t = [torch.from_numpy(np.ascontiguousarray(v)).cuda() for v in (p[..., 0], p[..., 1], g[..., 0], g[..., 1])]
        b.build_tokens_from_state(*t)
        ob.build_state(p[..., 0], p[..., 1], g[..., 0], g[..., 1])
        torch.cuda.synchronize()
        assert np.array_equal(b.tokens.cpu().numpy(), ob.tokens), (W, H, it)
        assert b.diagnostics.cpu().tolist() == ob.diagnostics.tolist(), (W, H, it)


@pytest.mark.parametrize("W,H,A,block", [(128, 96, 1100, True), (256, 128, 1300, False)])
def test_token_pass_beyond_1024_agents_matches_oracle(oracle, W, H, A, block):
    """More than 1024 agents (three workgroups per env of the token pass, ids
    past ten bits in the visible-agent keys) on a dense cell -> agent map
    (128 x 96, the agents on a block of consecutive cells, so most windows
    hold more than 13 of them) and on a sparse one (256 x 128, random
    cells), with a shared cell and an agent off the map: tokens and
    diagnostics equal the oracle's over two builds."""
    from iclr_2027_jointoom_amd import profile

    rng = np.random.default_rng(A + W)
    E = 2
    grids = (rng.random((E, W, H)) < 0.1).astype(np.int32)
    ext = profile(W, H)
    b = ext.MapfGPTObservationBuilder(torch.from_numpy(grids).cuda(), A)
    assert not b.single_launch
    ob = oracle.OracleMapfGPT(grids, A)
    goals = None
    for it in range(2):
        rows = np.zeros((E * A, 13), np.uint16)
        rows[:, 0] = np.repeat(np.arange(E), A)
        rows[:, 1] = np.tile(np.arange(A), E)
        for e in range(E):
            # dense case: a block of consecutive cells (whole map rows), so
            # windows there hold up to 121 agents; else distinct random cells
            if block:
                cells = rng.integers(0, W * H - A) + np.arange(A)
            else:
                cells = rng.permutation(W * H)[:A]
            rows[e * A:(e + 1) * A, 2] = cells // H
            rows[e * A:(e + 1) * A, 3] = cells % H
        if goals is None:
            goals = np.stack([rows[:, 2][::-1], rows[:, 3][::-1]], -1).copy()
        rows[:, 4:6] = goals
        rows[:, 6] = rng.integers(0, 5, E * A)
        rows[:, 7] = 1 if it == 0 else 0
        rows[:, 8:13] = rng.integers(0, 6, (E * A, 5))
        rows[3, 2:4] = rows[1030, 2:4]        # two agents on one cell
        rows[A + 1050, 2] = W + 1             # position off the map
        t = torch.from_numpy(rows.astype(np.int16)).cuda()
        b.build_tokens(t)
        ob.build_rows(rows)
        torch.cuda.synchronize()
        assert np.array_equal(b.tokens.cpu().numpy(), ob.tokens), it
        assert b.diagnostics.cpu().tolist() == ob.diagnostics.tolist(), it
    if block:
        # the visible-agent block is full for most egos
        assert (b.tokens[:, 121 + 12 * 10].cpu().numpy() != 66).mean() > 0.5


def test_raw_row_history_values_outside_action_range(oracle):
    """The reference emits 45 + value for any uint16 history value of a raw row."""
    grids, rows = _parity_fixture()
    rows[:, 8] = [0, 1, 2, 3, 4, 5, 6, 100, 210, 211, 255, 256, 4095, 40000, 65534, 65535][: len(rows)]
    ob = oracle.OracleMapfGPT(grids, 16)
    ob.build_rows(rows)
    ext = ext128()
    b = ext.MapfGPTObservationBuilder(torch.from_numpy(grids).cuda(), 16)
    b.build_tokens(torch.from_numpy(rows.astype(np.int16)).cuda())
    torch.cuda.synchronize()
    assert np.array_equal(b.tokens.cpu().numpy(), ob.tokens)
    assert ob.tokens.max() > 66  # the unbounded history tokens are really present


def _rows_case(rng, grids, A, goals=None):
    """Raw rows of every agent at distinct random cells (obstacles included);
    goals on free cells unless given."""
    E, W, H = grids.shape
    rows = np.zeros((E * A, 13), np.uint16)
    rows[:, 0] = np.repeat(np.arange(E), A)
    rows[:, 1] = np.tile(np.arange(A), E)
    for e in range(E):
        cells = rng.choice(W * H, A, replace=False)
        rows[e * A:(e + 1) * A, 2] = cells // H
        rows[e * A:(e + 1) * A, 3] = cells % H
        if goals is None:
            free = np.flatnonzero(grids[e].ravel() == 0)
            g = rng.choice(free, A, replace=False)
            rows[e * A:(e + 1) * A, 4] = g // H
            rows[e * A:(e + 1) * A, 5] = g % H
    if goals is not None:
        rows[:, 4:6] = goals
    rows[:, 6] = rng.integers(0, 5, E * A)
    rows[:, 8:13] = rng.integers(0, 6, (E * A, 5))
    return rows


@pytest.mark.parametrize("W,H,A", [(64, 64, 40), (36, 32, 40), (128, 32, 96), (64, 64, 1024), (32, 128, 77),
                                   (16, 256, 65)])
def test_single_launch_build_matches_oracle_and_two_launch_build(oracle, W, H, A):
    """Maps of at most 4096 cells with rows of at most 64 columns and at most
    1024 agents per env build in one launch: unpack, the env's field
    refreshes (with the greedy marks of the tiled copy) and tokens in one
    workgroup, diagnostics summed across workgroups.  Every output equals the
    oracle's and the two-launch build's (the same builder without its build
    scratch), over builds that keep, change and re-mark fields, with rejected
    rows, shared cells, positions off the map, goals on obstacles and agents
    on unreachable cells.  Marked maps of longer rows (32 x 128, 16 x 256)
    build in two launches with build scratch as without."""
    from iclr_2027_jointoom_amd import profile

    rng = np.random.default_rng(W + H + A)
    E = 3
    grids = (rng.random((E, W, H)) < 0.3).astype(np.int32)
    ext = profile(W, H)
    g = torch.from_numpy(grids).cuda()
    one = ext.MapfGPTObservationBuilder(g, A)
    two = ext.MapfGPTObservationBuilder(g, A)
    two._desc.build_scratch = None
    assert one.single_launch == (H <= 64) and not two.single_launch
    ob = oracle.OracleMapfGPT(grids, A)
    rows = _rows_case(rng, grids, A)
    goals = rows[:, 4:6].copy()
    diag_seen = np.zeros(4, np.int64)
    last_launch = 0
    for it in range(5):
        rows = _rows_case(rng, grids, A, goals)
        rows[:, 7] = 1 if it in (0, 3) else 0
        if it >= 1:
            rows[5, 0] = E + 1                     # rejected row (env out of range)
            rows[A + 2, 1] = A                     # rejected row (agent out of range)
            rows[7, 2:4] = rows[8, 2:4]            # two agents on one cell
            rows[2 * A + 1, 2] = W + 3             # position off the map
        if it == 2:
            obst = np.argwhere(grids[1] != 0)[0]
            rows[A + 5, 4:6] = obst                # goal on an obstacle
            rows[A + 6, 4:6] = (W + 1, 0)          # goal off the map
            rows[9, 4:6] = rows[10, 4:6]           # a changed goal
        t = torch.from_numpy(rows.astype(np.int16)).cuda()
        one.build_tokens(t)
        two.build_tokens(t)
        ob.build_rows(rows)
        torch.cuda.synchronize()
        for name in ("tokens", "labels", "active_mask", "cost_to_go", "state_packed", "histories",
                     "goal_cache", "diagnostics"):
            assert torch.equal(getattr(one, name), getattr(two, name)), (it, name)
        assert np.array_equal(one.tokens.cpu().numpy(), ob.tokens), it
        assert np.array_equal(one.cost_to_go.cpu().numpy(), ob.cost_to_go.view(np.int16)), it
        assert np.array_equal(one.state_packed.cpu().numpy(), ob.state_packed.view(np.int16)), it
        assert one.diagnostics.cpu().tolist() == ob.diagnostics.tolist(), it
        diag_seen += np.array(ob.diagnostics.tolist()) != 0
        # the number of this launch on this builder, derived on the device and
        # published after the clearing (uint64); a two-launch build leaves the
        # build scratch untouched
        if one.single_launch:
            last_launch += 1
        assert _published_launch(one) == last_launch, it
        # the resident builds of the same states agree as well
        st = one.state_packed.view(E, A, 8)
        if it == 4:
            one.build_tokens_from_state(*(st[:, :, k].contiguous() for k in (2, 3, 4, 5)))
            two.build_tokens_from_state(*(st[:, :, k].contiguous() for k in (2, 3, 4, 5)))
            torch.cuda.synchronize()
            for name in ("tokens", "active_mask", "cost_to_go", "diagnostics"):
                assert torch.equal(getattr(one, name), getattr(two, name)), name
    assert diag_seen[1] > 0 and diag_seen[2] > 0 and diag_seen[3] > 0
    greedy = ob.tokens[:, 121 + 9]
    assert len(np.unique(greedy)) > 4


def _published_launch(builder) -> int:
    return builder._build_scratch.cpu().view(torch.int64)[0].item()


def test_single_launch_build_replayed_from_a_graph_matches_two_launch_build():
    """A build captured into a graph keeps its single launch: every replay,
    over rows that change between replays (rejected rows, shared cells,
    positions off the map, a changed goal, resets), equals the eager
    two-launch build on every output, diagnostics included, and publishes a
    launch number one above the previous replay's.  Eager builds of the same
    builder run between replays."""
    from iclr_2027_jointoom_amd import profile

    W, H, A, E = 64, 64, 40, 3
    rng = np.random.default_rng(29)
    grids = (rng.random((E, W, H)) < 0.3).astype(np.int32)
    ext = profile(W, H)
    g = torch.from_numpy(grids).cuda()
    one = ext.MapfGPTObservationBuilder(g, A)
    two = ext.MapfGPTObservationBuilder(g, A)
    two._desc.build_scratch = None
    assert one.single_launch and not two.single_launch
    rows = _rows_case(rng, grids, A)
    goals = rows[:, 4:6].copy()
    static = torch.from_numpy(rows.astype(np.int16)).cuda()
    one.build_tokens(static)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    stream = torch.cuda.Stream()  # default priority
    stream.wait_stream(torch.cuda.current_stream())
    with torch.cuda.graph(graph, stream=stream):
        one.build_tokens(static)
    torch.cuda.current_stream().wait_stream(stream)
    torch.cuda.synchronize()
    launch = _published_launch(one)
    assert launch == 1
    diag_seen = np.zeros(4, np.int64)
    for it in range(6):
        rows = _rows_case(rng, grids, A, goals)
        rows[:, 7] = 1 if it in (0, 4) else 0
        if it % 2:
            rows[5, 0] = E + 1                     # rejected row (env out of range)
            rows[7, 2:4] = rows[8, 2:4]            # two agents on one cell
            rows[2 * A + 1, 2] = W + 3             # position off the map
        if it == 3:
            rows[9, 4:6] = rows[10, 4:6]           # a changed goal
        static.copy_(torch.from_numpy(rows.astype(np.int16)))
        if it == 2:
            one.build_tokens(static)               # an eager build between replays
            launch += 1
        graph.replay()
        launch += 1
        two.build_tokens(static)
        torch.cuda.synchronize()
        for name in ("tokens", "labels", "active_mask", "cost_to_go", "state_packed", "histories",
                     "goal_cache", "diagnostics"):
            assert torch.equal(getattr(one, name), getattr(two, name)), (it, name)
        assert _published_launch(one) == launch, it
        diag_seen += one.diagnostics.cpu().numpy() != 0
    assert diag_seen[1] > 0 and diag_seen[2] > 0 and diag_seen[3] > 0


def test_c2_full_size_build(oracle):
    """BASELINE C2/C3 shape (1024 envs x 128 agents, 64x64, p = 0.2) through
    three resident steps: the single-launch and the two-launch builds agree
    bit for bit on every output, three sampled envs equal the oracle, and
    every ego's own slot and window centre hold their closed-form tokens
    (relative position 0 -> 20, d - d = 0 -> 20, all egos reachable here)."""
    from iclr_2027_jointoom_amd import profile
    from iclr_2027_jointoom_amd.synthetic import make_batch

    E, W, A = 1024, 64, 128
    grids, starts, goals = make_batch(2027, E, W, W, A)
    ext = profile(W, W)
    g = torch.from_numpy(grids.astype(np.int32)).cuda()
    one = ext.MapfGPTObservationBuilder(g, A)
    two = ext.MapfGPTObservationBuilder(g, A)
    two._desc.build_scratch = None
    assert one.single_launch and not two.single_launch
    sim = ext.GridWorldSimulator(g, A, 0, E * W * W, 7, "standard_mapf", 512)
    sim.load_state(torch.from_numpy(starts).cuda(), torch.from_numpy(goals).cuda(),
                   torch.zeros((E, A), dtype=torch.uint8, device="cuda"),
                   torch.zeros(E, dtype=torch.int32, device="cuda"))
    sample = [0, 511, 1023]
    ob = oracle.OracleMapfGPT(grids[sample], A)
    gen = torch.Generator(device="cuda").manual_seed(5)
    for t in range(3):
        state = (sim.cur_x, sim.cur_y, sim.goal_x, sim.goal_y)
        one.build_tokens_from_state(*state)
        two.build_tokens_from_state(*state)
        ob.build_state(*(v.cpu().numpy()[sample] for v in state))
        torch.cuda.synchronize()
        for name in ("tokens", "active_mask", "cost_to_go", "state_packed", "labels", "goal_cache", "diagnostics"):
            assert torch.equal(getattr(one, name), getattr(two, name)), (t, name)
        assert one.diagnostics.cpu().tolist() == [0, 0, 0, 0]
        assert one.single_launch_waits_given_up == 0
        tok = one.tokens.view(E, A, 256)
        assert np.array_equal(tok[sample].cpu().numpy().reshape(-1, 256), ob.tokens), t
        assert bool((tok[:, :, 121] == 20).all() and (tok[:, :, 122] == 20).all()), t
        assert bool((tok[:, :, 60] == 20).all()), t
        acts = torch.randint(0, 5, (E, A), dtype=torch.uint8, device="cuda", generator=gen)
        one.append_actions(acts)
        two.append_actions(acts)
        ob.append(acts.cpu().numpy()[sample])
        sim.update_actions(acts)
        sim.step_sim_only()


def test_c5_full_size_build(oracle):
    """BASELINE C5 shape (256 envs x 1024 agents, 256x256 warehouses; sparse
    cell -> agent map, two 512-ego workgroups per env) through two resident
    steps: two sampled envs equal the oracle, and every ego's own slot and
    window centre hold their closed-form tokens."""
    from iclr_2027_jointoom_amd import profile
    from iclr_2027_jointoom_amd.synthetic import make_batch

    E, W, A = 256, 256, 1024
    grids, starts, goals = make_batch(2028, E, W, W, A, kind="warehouse")
    ext = profile(W, W)
    g = torch.from_numpy(grids.astype(np.int32)).cuda()
    b = ext.MapfGPTObservationBuilder(g, A)
    assert not b.single_launch
    sim = ext.GridWorldSimulator(g, A, 0, E * 1024, 7, "standard_mapf", 512)
    sim.load_state(torch.from_numpy(starts).cuda(), torch.from_numpy(goals).cuda(),
                   torch.zeros((E, A), dtype=torch.uint8, device="cuda"),
                   torch.zeros(E, dtype=torch.int32, device="cuda"))
    sample = [3, 250]
    ob = oracle.OracleMapfGPT(grids[sample], A)
    gen = torch.Generator(device="cuda").manual_seed(6)
    for t in range(2):
        state = (sim.cur_x, sim.cur_y, sim.goal_x, sim.goal_y)
        b.build_tokens_from_state(*state)
        ob.build_state(*(v.cpu().numpy()[sample] for v in state))
        torch.cuda.synchronize()
        assert b.diagnostics.cpu().tolist() == [0, 0, 0, 0]
        tok = b.tokens.view(E, A, 256)
        assert np.array_equal(tok[sample].cpu().numpy().reshape(-1, 256), ob.tokens), t
        assert bool((tok[:, :, 121] == 20).all() and (tok[:, :, 122] == 20).all()), t
        assert bool((tok[:, :, 60] == 20).all()), t
        acts = torch.randint(0, 5, (E, A), dtype=torch.uint8, device="cuda", generator=gen)
        b.append_actions(acts)
        ob.append(acts.cpu().numpy()[sample])
        sim.update_actions(acts)
        sim.step_sim_only()


def _late_diagnostic_rows(rng, grids, A, goals, envs):
    """Rows with a position off the map and two agents on one cell in each
    of ``envs`` (diagnostics [3] and [2] from those envs' workgroups only)."""
    E, W, H = grids.shape
    rows = _rows_case(rng, grids, A, goals)
    for e in envs:
        rows[e * A + 1, 2] = W + 2             # position off the map
        rows[e * A + 3, 2:4] = rows[e * A + 4, 2:4]  # two agents on one cell
    return rows


def test_single_launch_graph_replay_with_more_envs_than_arrival_classes():
    """130 envs (more workgroups than the 64 arrival classes, so classes hold
    two or three workgroups) with diagnostics only in envs 100..129: every
    replay of a captured single-launch build equals the two-launch build,
    diagnostics included, publishes the next launch number, and no
    workgroup's diagnostics wait gives up."""
    from iclr_2027_jointoom_amd import profile

    W, H, A, E = 64, 64, 24, 130
    rng = np.random.default_rng(130)
    grids = (rng.random((E, W, H)) < 0.2).astype(np.int32)
    ext = profile(W, H)
    g = torch.from_numpy(grids).cuda()
    one = ext.MapfGPTObservationBuilder(g, A)
    two = ext.MapfGPTObservationBuilder(g, A)
    two._desc.build_scratch = None
    assert one.single_launch and not two.single_launch
    goals = _rows_case(rng, grids, A)[:, 4:6].copy()
    static = torch.from_numpy(_late_diagnostic_rows(rng, grids, A, goals, range(100, 130)).astype(np.int16)).cuda()
    one.build_tokens(static)
    two.build_tokens(static)  # the same goal caches before the replays
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    stream = torch.cuda.Stream()  # default priority
    stream.wait_stream(torch.cuda.current_stream())
    with torch.cuda.graph(graph, stream=stream):
        one.build_tokens(static)
    torch.cuda.current_stream().wait_stream(stream)
    torch.cuda.synchronize()
    launch = _published_launch(one)
    for it in range(4):
        rows = _late_diagnostic_rows(rng, grids, A, goals, range(100 + it, 130, 3))
        static.copy_(torch.from_numpy(rows.astype(np.int16)))
        graph.replay()
        launch += 1
        two.build_tokens(static)
        torch.cuda.synchronize()
        for name in ("tokens", "labels", "active_mask", "cost_to_go", "state_packed", "histories",
                     "goal_cache", "diagnostics"):
            assert torch.equal(getattr(one, name), getattr(two, name)), (it, name)
        d = one.diagnostics.cpu().tolist()
        assert d[2] > 0 and d[3] > 0, d
        assert _published_launch(one) == launch, it
    assert one.single_launch_waits_given_up == 0


def test_single_launch_diagnostics_wait_gives_up_and_is_reported():
    """The bounded wait's give-up path, forced from the host: one arrival
    class's counter is advanced far ahead, so its workgroups derive a launch
    number that workgroup 0 never publishes.  Those with counts wait out the
    bound (milliseconds), add their counts anyway and are counted in the
    sticky word the builder reports; every kernel exits and the outputs
    equal the two-launch build's (the clear came first here)."""
    from iclr_2027_jointoom_amd import profile

    W, H, A, E = 32, 32, 16, 70
    rng = np.random.default_rng(70)
    grids = (rng.random((E, W, H)) < 0.2).astype(np.int32)
    ext = profile(W, H)
    g = torch.from_numpy(grids).cuda()
    one = ext.MapfGPTObservationBuilder(g, A)
    two = ext.MapfGPTObservationBuilder(g, A)
    two._desc.build_scratch = None
    goals = _rows_case(rng, grids, A)[:, 4:6].copy()
    rows = torch.from_numpy(_late_diagnostic_rows(rng, grids, A, goals, [1, 65]).astype(np.int16)).cuda()
    # class 1 (workgroups 1 and 65): uint64 arrival counter at word 32 + 1 * 32
    counters = one._build_scratch.view(torch.int64)
    counters[(32 + 32) // 2] = 1 << 40
    one.build_tokens(rows)
    two.build_tokens(rows)
    torch.cuda.synchronize()
    assert one.single_launch_waits_given_up == 2
    for name in ("tokens", "labels", "active_mask", "state_packed", "diagnostics"):
        assert torch.equal(getattr(one, name), getattr(two, name)), name
    one.clear_single_launch_waits()
    assert one.single_launch_waits_given_up == 0


def test_builds_from_two_streams_are_ordered():
    """A single-launch build issued from a second stream behind a long sleep,
    followed at once by a build on the current stream: the builder orders the
    second build after the first, so the outputs are the second build's (as
    the two-launch build issued in that order on one stream gives) and the
    launch numbers and diagnostics stay right."""
    from iclr_2027_jointoom_amd import profile

    W, H, A, E = 64, 64, 32, 6
    rng = np.random.default_rng(6)
    grids = (rng.random((E, W, H)) < 0.2).astype(np.int32)
    ext = profile(W, H)
    g = torch.from_numpy(grids).cuda()
    one = ext.MapfGPTObservationBuilder(g, A)
    two = ext.MapfGPTObservationBuilder(g, A)
    two._desc.build_scratch = None
    goals = _rows_case(rng, grids, A)[:, 4:6].copy()
    side = torch.cuda.Stream()  # default priority
    for it in range(3):
        rows_a = torch.from_numpy(_late_diagnostic_rows(rng, grids, A, goals, [1]).astype(np.int16)).cuda()
        rows_b = torch.from_numpy(_late_diagnostic_rows(rng, grids, A, goals, [4, 5]).astype(np.int16)).cuda()
        torch.cuda.synchronize()
        side.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(side):
            torch.cuda._sleep(20_000_000)
            one.build_tokens(rows_a)
        one.build_tokens(rows_b)
        two.build_tokens(rows_a)
        two.build_tokens(rows_b)
        torch.cuda.synchronize()
        for name in ("tokens", "labels", "active_mask", "state_packed", "diagnostics"):
            assert torch.equal(getattr(one, name), getattr(two, name)), (it, name)
        assert _published_launch(one) == 2 * (it + 1)
    assert one.single_launch_waits_given_up == 0


def test_single_launch_builds_over_moves_teleports_goal_changes_and_two_launch_refresh(oracle):
    """Single-launch builds over a run of one-cell moves (onto obstacles and off
    the map edges included), agents standing on their goal, teleports, goal
    changes and a two-launch refresh_distances between single-launch builds:
    every output equals the two-launch build's and the oracle's, so kept
    fields, their greedy marks and the windows of the tiled copies stay in
    step with what the builds rewrite."""
    from iclr_2027_jointoom_amd import profile

    E, W, A = 3, 64, 48
    rng = np.random.default_rng(77)
    grids = (rng.random((E, W, W)) < 0.3).astype(np.int32)
    ext = profile(W, W)
    g = torch.from_numpy(grids).cuda()
    one = ext.MapfGPTObservationBuilder(g, A)
    two = ext.MapfGPTObservationBuilder(g, A)
    two._desc.build_scratch = None
    assert one.single_launch and not two.single_launch
    ob = oracle.OracleMapfGPT(grids, A)
    pos = np.zeros((E, A, 2), np.int64)
    goal = np.zeros((E, A, 2), np.int64)
    for e in range(E):
        free = np.flatnonzero(grids[e].ravel() == 0)
        pick = rng.choice(free, 2 * A, replace=False)
        pos[e, :, 0], pos[e, :, 1] = pick[:A] // W, pick[:A] % W
        goal[e, :, 0], goal[e, :, 1] = pick[A:] // W, pick[A:] % W
    # a few agents start on their goal, on an obstacle, and on the map edges
    goal[0, 0] = pos[0, 0]
    pos[1, 1] = np.argwhere(grids[1] != 0)[0]
    pos[2, 2] = (0, 5)
    pos[2, 3] = (W - 1, W - 1)
    moves = np.array([[0, 0], [-1, 0], [1, 0], [0, -1], [0, 1]])
    dev = lambda a: torch.from_numpy(np.ascontiguousarray(a).astype(np.int16)).cuda()
    for t in range(8):
        if t == 3:
            pos[0, 5:9] = rng.integers(0, W, (4, 2))   # teleports
        if t == 4:
            goal[1, 10:14] = pos[1, 10:14]             # goals changed onto the agents' cells
        if t == 6:
            # fields rewritten by a two-launch pass between single-launch builds
            goal[2, 20:30] = rng.integers(0, W, (10, 2))
            state = [dev(pos[:, :, 0]), dev(pos[:, :, 1]), dev(goal[:, :, 0]), dev(goal[:, :, 1])]
            one.refresh_distances(*state)
            two.refresh_distances(*state)
        state = [dev(pos[:, :, 0]), dev(pos[:, :, 1]), dev(goal[:, :, 0]), dev(goal[:, :, 1])]
        one.build_tokens_from_state(*state)
        two.build_tokens_from_state(*state)
        ob.build_state(*(s.cpu().numpy() for s in state))
        torch.cuda.synchronize()
        for name in ("tokens", "active_mask", "cost_to_go", "state_packed", "labels", "goal_cache", "diagnostics"):
            assert torch.equal(getattr(one, name), getattr(two, name)), (t, name)
        assert np.array_equal(one.tokens.cpu().numpy(), ob.tokens), t
        # one-cell moves, clipped to [-1, W] so that some agents leave the map
        step = moves[rng.integers(0, 5, (E, A))]
        pos = np.clip(pos + step, -1, W)


def test_token_events_time_the_token_kernel_and_change_no_output():
    """token_events (a hipEvent_t pair in the descriptor) are recorded right
    before and after the token kernel, on the single-launch and the
    two-launch build alike: the builds with and without them agree bit for
    bit, and the pair spans a positive time no longer than the whole build
    bracketed from the host."""
    import ctypes

    from iclr_2027_jointoom_amd import profile

    rt = ctypes.CDLL("libamdhip64.so.7")
    rt.hipEventCreateWithFlags.argtypes = [ctypes.POINTER(ctypes.c_void_p), ctypes.c_uint]
    rt.hipEventElapsedTime.argtypes = [ctypes.POINTER(ctypes.c_float), ctypes.c_void_p, ctypes.c_void_p]
    rt.hipEventDestroy.argtypes = [ctypes.c_void_p]

    def event():
        ev = ctypes.c_void_p()
        assert rt.hipEventCreateWithFlags(ctypes.byref(ev), 0x20000000) == 0  # timing only, no system fence
        return ev.value

    rng = np.random.default_rng(11)
    E, W, A = 4, 64, 128
    grids = (rng.random((E, W, W)) < 0.2).astype(np.int32)
    ext = profile(W, W)
    g = torch.from_numpy(grids).cuda()
    rows = torch.from_numpy(_rows_case(rng, grids, A).astype(np.int16)).cuda()
    for single in (True, False):
        timed = ext.MapfGPTObservationBuilder(g, A)
        plain = ext.MapfGPTObservationBuilder(g, A)
        if not single:
            timed._desc.build_scratch = None
            plain._desc.build_scratch = None
        assert timed.single_launch == single
        evs = (event(), event())
        timed._desc.token_events[0], timed._desc.token_events[1] = evs
        try:
            for _ in range(2):
                host0, host1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
                host0.record()
                timed.build_tokens(rows)
                host1.record()
                plain.build_tokens(rows)
                torch.cuda.synchronize()
                ms = ctypes.c_float()
                assert rt.hipEventElapsedTime(ctypes.byref(ms), evs[0], evs[1]) == 0
                assert 0.0 < ms.value <= host0.elapsed_time(host1), (single, ms.value)
                for name in ("tokens", "labels", "active_mask", "cost_to_go", "state_packed", "histories",
                             "diagnostics"):
                    assert torch.equal(getattr(timed, name), getattr(plain, name)), (single, name)
        finally:
            timed._desc.token_events[0] = timed._desc.token_events[1] = None
            for ev in evs:
                rt.hipEventDestroy(ev)
