"""The sampler's host side and its oracle on the CPU, pinned by the
reference's own known answers: FlowShiftSchedule's ends and midpoint
(Tests/FlowSamplingTests.cs:12-24), the linspace and leading timesteps
(Tests/SchedulersTests.cs:28-52), a flow model's linspace run starting at
sigma 1 and ending at 0 (FlowSamplingTests.cs:50-58), and the Euler step
landing on the clean latent when the model predicts the exact velocity
(FlowSamplingTests.cs:60-80); the guidance combine at its closed forms."""

import numpy as np

import oracle
from naivediffusion_amd import sampling


def test_the_shifted_line_ends_at_one_and_bends_towards_noise():
    levels = sampling.FlowShiftSchedule(3.0)
    assert levels.train_timesteps == 1000
    assert abs(levels.sigma_max - 1.0) <= 1e-12
    assert abs(levels.sigma_min - 3 * 0.001 / (1 + 2 * 0.001)) <= 1e-12
    assert abs(levels.sigma_at(499) - 0.75) <= 1e-3
    assert abs(sampling.FlowShiftSchedule(1.0).sigma_at(499) - 0.5) <= 1e-12


def test_linspace_and_leading_timesteps():
    levels = sampling.FlowShiftSchedule(1.0)
    t, s = sampling.set_timesteps(levels, 5, "linspace")
    assert np.allclose(t, [999.0, 749.25, 499.5, 249.75, 0.0], atol=1e-9)
    assert s[-1] == 0 and len(s) == 6
    t, _ = sampling.set_timesteps(levels, 1, "linspace")
    assert list(t) == [999.0]
    t, _ = sampling.set_timesteps(levels, 20, "leading")
    assert list(t) == [951.0 - 50 * i for i in range(20)]


def test_a_flow_run_goes_from_noise_to_clean_data():
    """FlowSamplingTests.ASamplerRunsTheLineDownToCleanData: a model that
    knows x0 predicts noise - x0; eight Euler steps land on x0."""
    levels = sampling.FlowShiftSchedule(3.0)
    _, sigmas = sampling.set_timesteps(levels, 8, "linspace")
    assert sigmas[0] == np.float32(1.0) and sigmas[-1] == 0
    clean = np.array([0.3, -1.2, 2.0, 0.05], np.float32)
    sample = np.array([1.0, -0.5, 0.25, -2.0], np.float32)
    for step in range(8):
        sigma = sigmas[step]
        eps = (sample - (np.float32(1) - sigma) * clean) / sigma
        velocity = (eps - clean).astype(np.float32)
        # the prediction with no second branch is the velocity itself
        sample = oracle.euler_step(sample, velocity, sigma, sigmas[step + 1])
    assert np.max(np.abs(sample - clean)) <= 1e-4


def test_the_guidance_combine_closed_forms():
    g = np.random.default_rng(1)
    u, c = g.standard_normal(257).astype(np.float32), g.standard_normal(257).astype(np.float32)
    assert np.array_equal(oracle.cfg_combine(u, c, 0.0), u)
    assert np.max(np.abs(oracle.cfg_combine(u, c, 1.0) - c)) <= 1e-6 * np.max(np.abs(c)) * 4
    exp = u.astype(np.float64) + 4.5 * (c.astype(np.float64) - u)
    assert np.max(np.abs(oracle.cfg_combine(u, c, 4.5) - exp)) <= 1e-5 * np.max(np.abs(exp))
    # one rounding per float32 operation, the reference's order
    d = np.float32(c[0]) - np.float32(u[0])
    assert oracle.cfg_combine(u[:1], c[:1], 4.5)[0] == np.float32(u[0]) + np.float32(np.float32(4.5) * d)
