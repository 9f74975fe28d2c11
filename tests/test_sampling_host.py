"""The sampling around the decoders on the CPU: the generator against the C++ standard's known answer and the
reference build's libstdc++, the octree descent against the reference's own sample_anchors given the same logits
(bit for bit) and against closed forms, and the PLY writer against the reference's."""
import numpy as np
import pytest

import oracle as O
from conftest import GOLDEN
from decoders import MT19937_64, GaussianCloud, descend_octree, write_gaussian_ply


def test_mt19937_64_known_answer_and_libstdcxx_floats():
    # [rand.predef]: the 10000th output of a default-constructed mt19937_64 (seed 5489) is 9981545732273789042
    assert int(MT19937_64(5489).raw(10000)[-1]) == 9981545732273789042
    g = MT19937_64(7)
    u = g.uniform(100000)
    assert u.dtype == np.float32 and u.min() >= 0 and u.max() < 1
    assert abs(float(u.mean()) - 0.5) < 0.005
    if O.ref_available():
        for seed in (0, 1, 42, 2 ** 63 + 5):
            f, raw = O.ref_uniform_floats(seed, 5000)
            assert np.array_equal(MT19937_64(seed).raw(5000), raw)
            assert np.array_equal(MT19937_64(seed).uniform(5000), f)


def test_descent_closed_forms():
    # a certain child: every point goes to child 0 at every level, so all anchors lie in the corner cell
    certain = lambda c, r: np.tile(np.array([50.0, 0, 0, 0, 0, 0, 0, 0], np.float32), (c.shape[0], 1))  # noqa: E731
    p = descend_octree(certain, 300, 4, 3)
    assert p.shape == (300, 3) and np.all(p >= 0) and np.all(p < 1 / 16)
    # equal probabilities: systematic resampling gives each child n/8 points up to one
    flat = lambda c, r: np.zeros((c.shape[0], 8), np.float32)  # noqa: E731
    p = descend_octree(flat, 8000, 1, 5)
    child = (p[:, 0] >= 0.5).astype(int) + 2 * (p[:, 1] >= 0.5) + 4 * (p[:, 2] >= 0.5)
    assert np.all(np.abs(np.bincount(child, minlength=8) - 1000) <= 1)
    # the descent's centres: level l sees cells of side 2^-(l-1), centres at (coord + 0.5) / 2^(l-1)
    seen = []

    def record(c, r):
        seen.append((c.copy(), r))
        return np.zeros((c.shape[0], 8), np.float32)
    descend_octree(record, 64, 3, 1)
    assert [r for _, r in seen] == [2.0, 4.0, 8.0]
    assert np.array_equal(seen[0][0], np.full((1, 3), 0.5, np.float32))
    assert set(map(tuple, seen[1][0].tolist())) == {(a, b, c) for a in (0.25, 0.75) for b in (0.25, 0.75) for c in (0.25, 0.75)}
    with pytest.raises(ValueError, match="bad num_points or level"):
        descend_octree(flat, 0, 3, 1)
    with pytest.raises(ValueError, match="bad num_points or level"):
        descend_octree(flat, 10, 21, 1)


@pytest.mark.parametrize("num_points,level,seed", [(1, 1, 0), (100, 3, 7), (2048, 5, 11), (5000, 6, 1), (37, 8, 99)])
def test_descent_equals_the_reference_sampler_on_its_logits(num_points, level, seed):
    if not O.ref_available():
        pytest.skip("reference build absent (make -C oracle ref)")
    ref = O.RefDecoders(GOLDEN / "decoders_small")
    cond = np.random.default_rng(3).standard_normal((29, 16)).astype(np.float32)
    O.ref_lib().ref_set_quant_kernel(0)
    try:
        want = ref.sample_anchors(cond, num_points, level, seed)
        got = descend_octree(lambda c, r: ref.octree_logits(c, r, cond), num_points, level, seed)
    finally:
        O.ref_lib().ref_set_quant_kernel(-1)
        ref.close()
    assert np.array_equal(got, want)


def test_ply_writer_matches_the_reference(tmp_path):
    rng = np.random.default_rng(8)
    n = 257
    q = rng.standard_normal((n, 4)).astype(np.float32)
    cloud = {"xyz": rng.uniform(-0.5, 0.5, (n, 3)).astype(np.float32),
             "f_dc": rng.standard_normal((n, 3)).astype(np.float32),
             "scale": rng.uniform(1e-7, 0.1, (n, 3)).astype(np.float32),
             "rotation": (q / np.linalg.norm(q, axis=1, keepdims=True)).astype(np.float32),
             "opacity": np.concatenate([[0.0, 1.0], rng.uniform(0, 1, n - 2)]).astype(np.float32)}
    write_gaussian_ply(GaussianCloud(**cloud), tmp_path / "a.ply")
    data = (tmp_path / "a.ply").read_bytes()
    head, body = data.split(b"end_header\n")
    assert head.startswith(b"ply\nformat binary_little_endian 1.0\nelement vertex 257\n")
    rows = np.frombuffer(body, "<f4").reshape(n, 17)
    assert np.array_equal(rows[:, 1], -cloud["xyz"][:, 2]) and np.array_equal(rows[:, 2], cloud["xyz"][:, 1])
    if O.ref_available():
        O.ref_write_gaussian_ply(cloud, tmp_path / "b.ply")
        ref = (tmp_path / "b.ply").read_bytes()
        rhead, rbody = ref.split(b"end_header\n")
        assert rhead == head
        rrows = np.frombuffer(rbody, "<f4").reshape(n, 17)
        assert np.allclose(rows, rrows, rtol=2e-7, atol=2e-7)
