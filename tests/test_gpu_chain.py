"""GraphChain on the GPU: a three-link chain (Graph/GraphChain.cs) gives,
bit for bit, what the same expression gives built as one ModelBuilder
graph, its inputs converted to their declared types on the way in; a
chain whose result is an input passes it through an identity (:165-168);
and the oracle bounds the result at bf16 (2e-2)."""

import numpy as np
import pytest

import naivediffusion_amd as nd
import oracle
from naivediffusion_amd import GraphChain, rng
from naivediffusion_amd.layers import Layers
from naivediffusion_amd.tensors import HostDataType as DT, HostTensor
from conftest import rel_err

pytestmark = pytest.mark.gpu

T, D, F = 96, 128, 256


def normal(name, shape, std=1.0):
    return rng.normal(rng.tensor_seed(41, name), shape, 0.0, std)


def weights():
    return (HostTensor.FromFloats(normal("w1", (F, D), D ** -0.5)).ConvertTo(DT.BFloat16),
            HostTensor.FromFloats(normal("w2", (D, F), F ** -0.5)).ConvertTo(DT.BFloat16))


def body(model, x, w1, w2):
    h = Layers.Linear(model, Layers.Cast(x, DT.BFloat16), w1, activation="silu")
    return Layers.Linear(model, h, w2, residual=x)


def test_chain_matches_one_graph(device):
    print("[gpu] three-link chain vs one graph", flush=True)
    w1, w2 = weights()
    x = normal("x", (1, 1, T, D))

    c = GraphChain(device, DT.BFloat16)
    c.Input("x", [1, 1, T, D], DT.Float32)
    c.Set("h", Layers.Linear(c.Current, Layers.Cast(c.Get("x"), DT.BFloat16), w1, activation="silu"))
    c.Cut()
    c.Set("y", Layers.Linear(c.Current, c.Get("h"), w2, residual=c.Get("x")))
    c.Drop("h")
    c.Drop("x")
    c.Cut()
    c.Set("y", Layers.Cast(c.Get("y"), DT.Float32))
    c.Finish("y")
    assert c.LinkCount == 3 and c.StreamedBytes == 0
    assert c.PersistentBytes >= 2 * F * D * 2 and c.ResidentBytes == c.PersistentBytes
    # An fp16 tensor for an fp32 input is converted on the way in.
    got = c.Run({"x": HostTensor.FromFloats(x).ConvertTo(DT.Float16)}).ToFloats()
    c.Dispose()

    m = nd.ModelBuilder(device, DT.BFloat16)
    xin = m.Placeholder([1, 1, T, D], DT.Float32)
    m.Compile([Layers.Cast(body(m, xin, w1, w2), DT.Float32)])
    x16 = HostTensor.FromFloats(x).ConvertTo(DT.Float16).ConvertTo(DT.Float32)
    want = m.Run(x16)[0].ToFloats()
    m.Dispose()
    assert np.array_equal(got, want)

    xf = x16.ToFloats().reshape(T, D)
    xb = HostTensor.FromFloats(xf).ConvertTo(DT.BFloat16).ToFloats().reshape(T, D)
    h = oracle.silu(xb @ w1.ToFloats().reshape(F, D).T)
    ref = xf + h @ w2.ToFloats().reshape(D, F).T
    assert rel_err(got.reshape(T, D), ref) <= 2e-2


def test_chain_result_may_be_an_input(device):
    c = GraphChain(device, DT.Float32)
    c.Input("x", [1, 1, 4, 8])
    c.Finish("x")
    x = normal("px", (1, 1, 4, 8))
    got = c.Run({"x": HostTensor.FromFloats(x)}).ToFloats()
    c.Dispose()
    assert np.array_equal(got.reshape(x.shape), x)


def test_chain_run_checks_inputs(device):
    c = GraphChain(device, DT.Float32)
    c.Input("x", [1, 1, 4, 8])
    c.Set("y", Layers.Silu(c.Get("x")))
    c.Finish("y")
    with pytest.raises(nd.ArgumentError, match="z is not an input of this chain"):
        c.Run({"x": HostTensor.FromFloats(normal("cx", (1, 1, 4, 8))), "z": HostTensor.FromFloats(np.zeros(1))})
    with pytest.raises(nd.InvalidOperationError, match="x was not supplied"):
        c.Run({})
    c.Dispose()
