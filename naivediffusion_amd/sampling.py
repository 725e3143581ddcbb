"""The sampling loop around the denoiser with the latent resident on the GPU.

The reference's loop (Pipeline/GenerationPipeline.cs:576-616) uploads the
latent, runs Predict once per guidance branch, downloads every prediction,
combines them on the CPU (Pipeline/GuidanceStrategy.cs:34-66) and takes the
sampler's step on the CPU (Sampling/Schedulers.cs). Here the predictions and
the latent stay in HBM: the guidance combine and the Euler step are one
kernel (ndx_op_guided_euler_step) with the step's scalars read on the device,
and only the finished latent comes back.

The noise levels follow the reference for the flow models (rectified flow,
FlowShiftSchedule, Sampling/NoiseSchedule.cs:147-170) with its linspace and
leading spacings (Schedulers.cs:92-137).
"""

from __future__ import annotations

from typing import Callable, List, Sequence

import numpy as np

from .graph import CompiledModel, Graph, Ops
from .tensors import Device, DeviceTensor, HostDataType, HostTensor

F32 = HostDataType.Float32


class FlowShiftSchedule:
    """FlowShiftSchedule (NoiseSchedule.cs:147-170): at training timestep i
    (t = (i + 1) / T) the level is shift * t / (1 + (shift - 1) t); 1 at the
    top."""

    def __init__(self, shift: float = 3.0, train_timesteps: int = 1000):
        t = (np.arange(train_timesteps, dtype=np.float64) + 1.0) / train_timesteps
        self.train_sigmas = shift * t / (1.0 + (shift - 1.0) * t)

    @property
    def train_timesteps(self) -> int:
        return len(self.train_sigmas)

    @property
    def sigma_min(self) -> float:
        return float(self.train_sigmas[0])

    @property
    def sigma_max(self) -> float:
        return float(self.train_sigmas[-1])

    def sigma_at(self, timestep: float) -> float:
        """NoiseSchedule.SigmaAt (:73-80): linear between training levels."""
        s = self.train_sigmas
        low = int(np.clip(np.floor(timestep), 0, len(s) - 1))
        high = min(low + 1, len(s) - 1)
        return float(s[low] + (s[high] - s[low]) * (timestep - low))


def set_timesteps(levels: FlowShiftSchedule, steps: int, spacing: str = "linspace"):
    """SigmaScheduler.SetTimesteps (Schedulers.cs:92-137) for the linspace
    and leading spacings: (timesteps float64 [steps], sigmas float32
    [steps + 1], the last 0)."""
    T = levels.train_timesteps
    if spacing == "linspace":
        if steps == 1:
            timesteps = np.array([T - 1], np.float64)
        else:
            timesteps = (T - 1) * (1.0 - np.arange(steps, dtype=np.float64) / (steps - 1))
    elif spacing == "leading":
        stride = T // steps
        timesteps = np.array([(steps - 1 - i) * stride + 1 for i in range(steps)], np.float64)
    else:
        raise ValueError(f"unknown spacing {spacing!r}")
    sigmas = np.zeros(steps + 1, np.float32)
    for i, t in enumerate(timesteps):
        sigmas[i] = np.float32(levels.sigma_at(float(t)))
    return timesteps, sigmas


class GuidedEulerStep:
    """One sampler step as a compiled model on the device: (x, [uncond,]
    cond, scalars) -> x + (u + g (c - u)) (sigma_next - sigma)."""

    def __init__(self, device: Device, shape: Sequence[int], branches: int):
        if branches not in (1, 2):
            raise ValueError("one branch (no guidance) or two (negative first)")
        self.device, self.branches = device, branches
        g = Graph(device)
        x = g.Input(F32, list(shape))
        u = g.Input(F32, list(shape)) if branches == 2 else None
        c = g.Input(F32, list(shape))
        s = g.Input(F32, [1, 1, 1, 4])
        self.model = CompiledModel(g, [Ops.GuidedEulerStep(x, u, c, s)], device)
        g.Dispose()
        self.scalars: List[DeviceTensor] = []

    def Prepare(self, guidance: float, sigmas: np.ndarray) -> None:
        """Uploads every step's (g, sigma, sigma_next) once, so the steps
        queue without waiting on the host."""
        self.Release()
        self.scalars = [self.device.Upload(HostTensor.FromFloats(
            np.array([guidance, sigmas[i], sigmas[i + 1], 0.0], np.float32), 1, 1, 1, 4))
            for i in range(len(sigmas) - 1)]

    def Step(self, step: int, x: DeviceTensor, predictions: List[DeviceTensor], out: DeviceTensor) -> None:
        """Queues step `step` into out (another tensor than x)."""
        if len(predictions) != self.branches:
            raise ValueError(f"{self.branches} predictions expected")
        self.model.DispatchInto([x, *predictions, self.scalars[step]], [out])

    def Release(self):
        for t in self.scalars:
            t.Dispose()
        self.scalars = []

    def Dispose(self):
        self.Release()
        self.model.Dispose()


def sample(device: Device, predict: Callable[[DeviceTensor, int], List[DeviceTensor]], latent: DeviceTensor,
           sigmas: np.ndarray, guidance: float, branches: int) -> DeviceTensor:
    """The loop of GenerationPipeline (:576-616) for a flow model and the Euler
    sampler, the latent on the device throughout: per step, predict(x, step)
    queues the branches' predictions (negative first) and returns them as
    device tensors, and one kernel combines them and steps x; nothing waits
    on the host until the end. Returns the final latent (a new tensor;
    `latent` is left as it was)."""
    steps = len(sigmas) - 1
    if steps < 1:
        raise ValueError("at least one step")
    stepper = GuidedEulerStep(device, latent.Shape, branches)
    stepper.Prepare(guidance, sigmas)
    buf = [device.Empty(F32, latent.Shape), device.Empty(F32, latent.Shape)]
    x = latent
    for step in range(steps):
        preds = predict(x, step)
        stepper.Step(step, x, preds, buf[step % 2])
        x = buf[step % 2]
    device.Synchronize()
    stepper.Dispose()
    buf[steps % 2].Dispose()
    return x
