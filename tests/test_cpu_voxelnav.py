"""The oracle's VoxelNav (examples/VoxelNav/voxelnav.metal:9-174) pinned against
what the reference's text fixes, independently of the oracle's code: the RNG
draw count and the terrain rebuilt in float64 from the same draws; the depth
camera on flat ground, where the geometry gives each ray's hit in closed form;
and the move, cobble, reward and termination rules on constructed states."""
import math

import numpy as np
import pytest

VOXELNAV = 4
W = 32
HEADER = 32  # x, z, yaw, gx, gz, prevDist (f32), steps, cobble (u32)
SIZE = HEADER + W * W


def xorshift(s):
    s ^= (s << 13) & 0xFFFFFFFF
    s ^= s >> 17
    s ^= (s << 5) & 0xFFFFFFFF
    return s


def draws(seed, k):
    out, s = [], seed
    for _ in range(k):
        s = xorshift(s)
        out.append(s)
    return out, s


def unpack(st):
    f = st[:24].view(np.float32)
    u = st[24:32].view(np.uint32)
    return dict(x=f[0], z=f[1], yaw=f[2], gx=f[3], gz=f[4], prev=f[5], steps=int(u[0]), cobble=int(u[1]),
                height=st[HEADER:].reshape(W, W))


def make_state(height, x, z, yaw, gx, gz, steps=0, cobble=16):
    st = np.zeros(SIZE, np.uint8)
    prev = np.float32(math.sqrt((gx - x) ** 2 + (gz - z) ** 2))
    st[:24] = np.array([x, z, yaw, gx, gz, prev], np.float32).view(np.uint8)
    st[24:32] = np.array([steps, cobble], np.uint32).view(np.uint8)
    st[HEADER:] = np.asarray(height, np.uint8).ravel()
    return st


def step(orc, st, action):
    a = np.array([action], np.int32)
    obs, r, d = np.zeros(40, np.float32), np.zeros(1, np.float32), np.zeros(1, np.uint8)
    orc.lib().orc_env_step(VOXELNAV, orc.ptr(st), orc.ptr(a), orc.ptr(obs), orc.ptr(r), orc.ptr(d))
    return obs, float(r[0]), int(d[0])


def test_env_info(orc):
    i = orc.env_info(VOXELNAV)
    assert (i.state_bytes, i.obs_dim, i.act_dim, i.continuous) == (SIZE, 40, 6, 0)


@pytest.mark.parametrize("seed", [1, 7, 12345, 2654435761 + 1, 0xDEADBEEF])
def test_reset_terrain_spawn_and_draws(orc, seed):
    st = np.zeros(SIZE, np.uint8)
    rng = np.array([seed], np.uint32)
    orc.lib().orc_env_reset(VOXELNAV, orc.ptr(st), orc.ptr(rng))
    d, last = draws(seed, 33)  # 25 knots, width, left, lift, x, z, gx, gz, yaw
    assert int(rng[0]) == last, "reset takes 33 draws"
    u = [(v >> 8) / 16777216.0 for v in d]
    knot = [3.0 + 6.0 * u[i] for i in range(25)]
    width, left, lift = 2 + d[25] % 4, 12 + d[26] % 6, d[27] % 3
    s = unpack(st)
    h = s["height"]
    mism = 0
    for cx in range(W):
        fx = cx / 31 * 4
        ix = min(int(fx), 3)
        tx = fx - ix
        for cz in range(W):
            fz = cz / 31 * 4
            iz = min(int(fz), 3)
            tz = fz - iz
            lo = knot[ix * 5 + iz] + (knot[(ix + 1) * 5 + iz] - knot[ix * 5 + iz]) * tx
            hi = knot[ix * 5 + iz + 1] + (knot[(ix + 1) * 5 + iz + 1] - knot[ix * 5 + iz + 1]) * tx
            v = lo + (hi - lo) * tz
            want = math.floor(v + 0.5)
            if left <= cx < left + width:
                want = 0
            elif cx >= left + width:
                want = min(want + lift, 15)
            if h[cx, cz] != want:
                # float32 and float64 may round differently only at a .5 tie
                assert abs(v - math.floor(v) - 0.5) < 1e-4, (cx, cz, h[cx, cz], want, v)
                mism += 1
    assert mism <= 2
    # spawn on the near side, goal beyond the chasm, both inside the map
    assert 2.5 <= s["x"] < 2.5 + (left - 4) and 2.5 <= s["z"] < 2.5 + 27
    assert left + width + 2.5 <= s["gx"] < 29.5 and 2.5 <= s["gz"] < 29.5
    assert h[int(s["x"]), int(s["z"])] > 0 and h[int(s["gx"]), int(s["gz"])] > 0
    assert abs(s["x"] - (2.5 + u[28] * (left - 4))) < 1e-5 and abs(s["gz"] - (2.5 + u[31] * 27)) < 1e-5
    assert -math.pi <= s["yaw"] < math.pi and abs(s["yaw"] - (-math.pi + 2 * math.pi * u[32])) < 1e-5
    assert s["steps"] == 0 and s["cobble"] == 16
    assert abs(s["prev"] - math.hypot(s["gx"] - s["x"], s["gz"] - s["z"])) < 1e-5


def exit_depth(x, z, dx, dz):
    """First t on the 0.5 grid whose sample leaves the map (flat ground below eye)."""
    t = 0.5
    while t < 24.0:
        if not (0 <= math.floor(x + t * dx) < W and 0 <= math.floor(z + t * dz) < W):
            return t
        t += 0.5
    return 24.0


@pytest.mark.parametrize("yaw", [0.0, 0.7, -2.0])
def test_camera_on_flat_ground(orc, yaw):
    x, z, ground = 16.25, 15.75, 5
    st = make_state(np.full((W, W), ground), x, z, yaw, 28.0, 27.0)
    obs, r, d = step(orc, st, 9)  # not an action: only the clock and the camera move
    fov = math.pi / 2
    for c in range(8):
        a = yaw + (c / 7 - 0.5) * fov
        for row, pitch in enumerate((-45.0, -20.0, 0.0, 15.0)):
            p = math.radians(pitch)
            if pitch < 0:
                # eye 1.6 above the ground: first grid t with 1.6 + t sin p <= 0
                t = math.ceil(1.6 / -math.sin(p) / 0.5) * 0.5
            else:
                t = exit_depth(x, z, math.cos(p) * math.cos(a), math.cos(p) * math.sin(a))
            assert obs[c * 4 + row] == pytest.approx(t / 24.0, abs=1e-7), (c, pitch)
    gx, gz = 28.0 - x, 27.0 - z
    np.testing.assert_allclose(obs[32:40], [(gx * math.cos(yaw) + gz * math.sin(yaw)) / 32,
                                            (-gx * math.sin(yaw) + gz * math.cos(yaw)) / 32, 0.0,
                                            math.hypot(gx, gz) / 32, math.sin(yaw), math.cos(yaw), 1.0,
                                            ground / 16], atol=2e-6)
    assert r == pytest.approx(-0.05, abs=1e-7) and d == 0 and unpack(st)["steps"] == 1


def corridor(heights_along_x):
    """Terrain that varies along x only (same height for every z)."""
    h = np.zeros((W, W), np.uint8)
    for cx, v in enumerate(heights_along_x):
        h[cx, :] = v
    return h


def test_moves_climb_block_fall_and_jump(orc):
    prof = [4] * W
    prof[11], prof[12], prof[14] = 5, 7, 0  # one up, two up, void
    # yaw 0 faces +x: one block up is climbable
    st = make_state(corridor(prof), 10.5, 8.5, 0.0, 30.5, 8.5)
    obs, r, d = step(orc, st, 0)
    s = unpack(st)
    assert s["x"] == np.float32(11.5) and d == 0 and r == pytest.approx(-0.05 + 0.2 * 1.0, abs=1e-6)
    # two blocks up: blocked, position unchanged, no progress
    obs, r, d = step(orc, st, 0)
    assert unpack(st)["x"] == np.float32(11.5) and r == pytest.approx(-0.05, abs=1e-6)
    # back (action 1) moves -x
    step(orc, st, 1)
    assert unpack(st)["x"] == np.float32(10.5)
    # from x = 13.5 a step forward lands in the void at 14.5: fell, -5, done
    st = make_state(corridor(prof), 13.5, 8.5, 0.0, 30.5, 8.5)
    obs, r, d = step(orc, st, 0)
    assert unpack(st)["x"] == np.float32(14.5) and d == 1
    assert r == pytest.approx(-0.05 + 0.2 * 1.0 - 5.0, abs=1e-5)
    # a jump (action 4) moves two cells and clears the void
    st = make_state(corridor(prof), 13.5, 8.5, 0.0, 30.5, 8.5)
    obs, r, d = step(orc, st, 4)
    assert unpack(st)["x"] == np.float32(15.5) and d == 0
    assert r == pytest.approx(-0.05 + 0.2 * 1.5, abs=1e-5)  # progress 2 clamped to 1.5
    # leaving the map is refused
    st = make_state(corridor([4] * W), 31.5, 8.5, 0.0, 2.5, 8.5)
    step(orc, st, 0)
    assert unpack(st)["x"] == np.float32(31.5)


def test_turns_wrap_yaw(orc):
    st = make_state(corridor([4] * W), 8.5, 8.5, 3.0, 30.5, 30.5)
    step(orc, st, 3)  # 3 + pi/6 > pi wraps to 3 + pi/6 - 2 pi
    assert unpack(st)["yaw"] == pytest.approx(3.0 + math.pi / 6 - 2 * math.pi, abs=1e-5)
    step(orc, st, 2)
    step(orc, st, 2)
    assert unpack(st)["yaw"] == pytest.approx(3.0 - math.pi / 6, abs=1e-5)


def test_cobble_placement(orc):
    prof = [4] * W
    prof[9], prof[10] = 0, 6
    st = make_state(corridor(prof), 8.5, 3.5, 0.0, 30.5, 3.5)
    step(orc, st, 5)  # the cell ahead is void: filled to the agent's height
    s = unpack(st)
    assert s["height"][9, 3] == 4 and s["cobble"] == 15 and s["height"][9, 4] == 0
    step(orc, st, 5)  # now level with the agent: raised by one
    s = unpack(st)
    assert s["height"][9, 3] == 5 and s["cobble"] == 14
    step(orc, st, 5)  # one above the agent: unchanged
    s = unpack(st)
    assert s["height"][9, 3] == 5 and s["cobble"] == 14
    st = make_state(corridor(prof), 8.5, 3.5, 0.0, 30.5, 3.5, cobble=0)
    step(orc, st, 5)  # no cobble left
    assert unpack(st)["height"][9, 3] == 0
    st = make_state(corridor(prof), 31.5, 3.5, 0.0, 2.5, 3.5)
    step(orc, st, 5)  # the cell ahead is outside the map
    assert unpack(st)["cobble"] == 16


def test_goal_and_step_cap(orc):
    st = make_state(corridor([4] * W), 10.5, 8.5, 0.0, 12.0, 8.5)
    obs, r, d = step(orc, st, 0)  # to 11.5: distance 0.5 < 1.5
    assert d == 1 and r == pytest.approx(-0.05 + 0.2 * 1.0 + 10.0, abs=1e-5)
    st = make_state(corridor([4] * W), 10.5, 8.5, 0.0, 30.5, 30.5, steps=249)
    obs, r, d = step(orc, st, 2)
    assert d == 1 and unpack(st)["steps"] == 250
    st = make_state(corridor([4] * W), 10.5, 8.5, 0.0, 30.5, 30.5, steps=247)
    assert step(orc, st, 2)[2] == 0


def test_random_rollout_statistics(orc):
    """Long random rollouts stay in range: depths in (0, 1], finite features,
    rewards from the shaping formula's range, episodes end."""
    g = orc.GymState(VOXELNAV, 256, 3)
    acts, obs, rew, dn = orc.rollout(g, 300, random=True, threads=4)
    assert np.all((obs[..., :32] > 0) & (obs[..., :32] <= 1.0)) and np.isfinite(obs).all()
    assert rew.min() >= -0.05 - 0.3 - 5.0 - 1e-5 and rew.max() <= -0.05 + 0.3 + 10.0 + 1e-5
    assert dn.sum() > 256  # every env ended at least once (cap 250) on average
    assert set(np.unique(acts)) == set(range(6))
