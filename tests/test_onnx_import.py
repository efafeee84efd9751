"""The ONNX importer (harness/onnx_import.py): the protobuf wire format it decodes, and the
graphs it builds, checked against torch's forward pass of the same networks (the ONNX
bytes come from tests/onnx_writer.py, node for node as an exporter writes them) and
against the op sequence the harness's own ResNet-18 builder lowers to."""
import numpy as np
import pytest

from harness import lowering as LW
from harness import models
from harness import onnx_import as OI
from oracle import golden as G

import onnx_writer as W
import torch_onnx_nets as N


def test_wire_format_tensors_and_attributes():
    m = W.Model(13)
    f32 = np.arange(-6, 6, dtype=np.float32).reshape(3, 4) / 7
    i64 = np.array([[-3, 0, 2 ** 40]], np.int64)
    f16 = np.array([1.5, -2.25, 65504.0], np.float16)
    m.inits.append(W.tensor("f32_raw", f32))
    m.inits.append(W.tensor("f32_field", f32, raw=False))
    m.inits.append(W.tensor("i64_raw", i64))
    m.inits.append(W.tensor("i64_field", i64, raw=False))
    m.inits.append(W.tensor("f16", f16))
    m.inits.append(W.tensor("scalar", np.array(2.5, np.float32)))
    m.node("Foo", ["a", "", "b"], n_out=2, i=-7, f=0.25, s="text", ints=[3, -1, 2 ** 33], floats=[0.5, -1.0],
           t=np.array([[1, 2]], np.int32))
    m.input("a", (2, "batch", 5))
    m.output("foo1_0", (4,))
    r = OI.read_model(m.bytes())
    assert r["opset"] == 13
    inits = r["initializers"]
    for name, want in (("f32_raw", f32), ("f32_field", f32), ("i64_raw", i64), ("i64_field", i64), ("f16", f16),
                       ("scalar", np.array(2.5, np.float32))):
        assert inits[name].dtype == want.dtype and inits[name].shape == want.shape
        assert np.array_equal(inits[name], want)
    (n,) = r["nodes"]
    assert n["op_type"] == "Foo" and n["input"] == ["a", "", "b"] and n["output"] == ["foo1_0", "foo1_1"]
    a = n["attrs"]
    assert a["i"] == -7 and a["f"] == 0.25 and a["s"] == b"text" and a["ints"] == [3, -1, 2 ** 33]
    assert a["floats"] == [0.5, -1.0] and np.array_equal(a["t"], np.array([[1, 2]], np.int32))
    assert r["inputs"] == [("a", 1, [2, None, 5])] and r["outputs"] == [("foo1_0", 1, [4])]


def test_unsupported_operator_and_symbolic_input():
    m = W.Model(13)
    x = m.input("x", ("n", 4))
    m.output(m.node("LpNormalization", [x]), ("n", 4))
    with pytest.raises(OI.OnnxImportError, match="symbolic"):
        OI.import_model(m.bytes())
    with pytest.raises(OI.OnnxImportError, match="LpNormalization"):
        OI.import_model(m.bytes(), {"x": (2, 4)})


@pytest.mark.parametrize("opset", [10, 13])
def test_edge_net_matches_torch(opset):
    """Conv bias / dilation / depthwise / asymmetric pads, BN, Clip (both opset forms),
    ceil-mode MaxPool, the Shape-Gather-Unsqueeze-Concat flatten, Gemm alpha/beta."""
    import torch
    forward, data = N.edge_net(3, opset)
    g = OI.import_model(data)
    kinds = [op.kind for op in g.compute_ops()]
    assert kinds.count("pad") == 2 and kinds.count("conv2d") == 3 and "maxpool2d" in kinds
    x = np.random.default_rng(0).standard_normal((3, 3, 9, 9)).astype(np.float32)
    (got,) = G.run_graph(g, {"x": x})
    with torch.no_grad():
        want = forward(torch.from_numpy(x)).numpy()
    np.testing.assert_allclose(got, want, rtol=1e-4, atol=1e-5 * np.abs(want).max())


def test_resnet18_matches_torch():
    import torch
    net, data = N.resnet18(2)
    g = OI.import_model(data)
    x = np.random.default_rng(1).uniform(0, 1, (2, 3, 224, 224)).astype(np.float32)
    (got,) = G.run_graph(g, {"x": x})
    with torch.no_grad():
        want = net(torch.from_numpy(x)).numpy()
    np.testing.assert_allclose(got, want, rtol=1e-3, atol=1e-4 * np.abs(want).max())


def test_mobilenet_v2_matches_torch():
    """The torchvision-layout MobileNetV2 (depthwise groups, ReLU6 as Clip, residual adds)
    imports to a graph whose f32 forward pass is torch's."""
    import torch
    net, data = N.mobilenet_v2(2)
    g = OI.import_model(data)
    kinds = [op.kind for op in g.compute_ops()]
    assert kinds.count("conv2d") == 52 and kinds.count("add") >= 10
    x = np.random.default_rng(2).uniform(0, 1, (2, 3, 224, 224)).astype(np.float32)
    (got,) = G.run_graph(g, {"x": x})
    with torch.no_grad():
        want = net(torch.from_numpy(x)).numpy()
    np.testing.assert_allclose(got, want, rtol=1e-3, atol=1e-4 * np.abs(want).max())


def test_resnet18_lowers_like_the_builder():
    """The imported ResNet-18 and the harness's builder (BN as mul + add, the importer's
    layout) lower to the same W8A8 op sequence: 20 q-convolutions and one q-matmul with the
    same epilogues, the pad + max pool, the global average pool."""
    _, data = N.resnet18(2)
    imported = LW.prepare(OI.import_model(data))
    built = LW.prepare(models.resnet18(batch=2, bn_epilogue=True))
    for g in (imported, built):
        LW.w8a8(g, peaks=LW.calibrate(g, [{"x": models.image_batch((2, 3, 224, 224), 11)}]))

    def shape_of(g):
        return [(op.kind, tuple(op.result.type.shape), tuple(s[0] for s in op.attrs.get("epilogue", ())))
                for op in g.compute_ops()]

    assert shape_of(imported) == shape_of(built)
    kinds = [k for k, _, _ in shape_of(imported)]
    assert kinds.count("qconv2d") == 20 and kinds.count("qmatmul") == 1
