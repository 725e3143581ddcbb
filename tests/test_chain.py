"""GraphChain's bookkeeping (Graph/GraphChain.cs) on a device-less graph:
declared inputs become placeholders when first read and only then, named
values replace one another, dropped values are gone, and every misuse the
reference rejects is rejected with its message (:88-90, :106-108,
:127-130, :144-146, :208-211, :222-224)."""

import pytest

import naivediffusion_amd as nd
from naivediffusion_amd import GraphChain, Ops
from naivediffusion_amd.layers import Layers
from naivediffusion_amd.tensors import HostDataType as DT


def chain():
    return GraphChain(None, DT.BFloat16)


def test_inputs_are_read_lazily_and_in_order():
    c = chain()
    c.Input("a", [1, 1, 8, 16])
    c.Input("b", [1, 1, 8, 16], DT.Float32)
    c.Input("unused", [1, 1, 1, 1], DT.Int32)
    assert c.Current._placeholders == []
    b = c.Get("b")
    a = c.Get("a")
    assert c.Get("b") is b  # read again: the same value, no second placeholder
    assert c._placeholders == ["b", "a"]
    assert a.DataType == DT.BFloat16 and b.DataType == DT.Float32
    assert c.Shape("a") == [1, 1, 8, 16]
    assert len(c.Current._placeholders) == 2


def test_set_replaces_and_carries_shape():
    c = chain()
    c.Input("x", [1, 1, 4, 32])
    x = c.Get("x")
    c.Set("y", Layers.Cast(x, DT.Float32))
    assert c.Shape("y") == [1, 1, 4, 32]
    c.Cut()
    c.Set("y", Ops.Reinterpret(c.Get("y"), [1, 1, 8, 16]))
    assert c.Shape("y") == [1, 1, 8, 16]
    assert c.Get("y").DataType == DT.Float32
    assert c.LinkCount == 1


def test_drop_removes_the_value():
    c = chain()
    c.Input("x", [1, 1, 4, 32])
    c.Get("x")
    c.Drop("x")
    with pytest.raises(nd.ArgumentError, match="x has not been produced yet"):
        c.Get("x")
    with pytest.raises(nd.ArgumentError, match="x is not a live value"):
        c.Drop("x")


def test_misuse_is_rejected():
    c = chain()
    c.Input("x", [1, 1, 4, 32])
    with pytest.raises(nd.ArgumentError, match="x was declared twice"):
        c.Input("x", [1, 1, 4, 32])
    with pytest.raises(nd.ArgumentError, match="nothing has not been produced yet"):
        c.Get("nothing")
    other = nd.Graph(None, DT.BFloat16)
    with pytest.raises(nd.ArgumentError, match="y belongs to an earlier link"):
        c.Set("y", other.Input(DT.BFloat16, [1, 1, 4, 32]))
    with pytest.raises(nd.InvalidOperationError, match=r"Finish\(\) the chain before running it"):
        c.Run({})
    with pytest.raises(nd.ArgumentError, match="gone is not a live value at the end"):
        c.Finish("gone")
    other.Dispose()
    c.Dispose()


def test_byte_counts_before_finish():
    c = chain()
    assert (c.PersistentBytes, c.StreamedBytes, c.ResidentBytes, c.TemporaryBytes, c.LinkCount) == (0, 0, 0, 0, 0)
