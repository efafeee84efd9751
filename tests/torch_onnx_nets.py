"""Test infrastructure: torch networks (random weights, eval mode) and the ONNX models an
exporter would write for them, node for node (tests/onnx_writer.py), so the importer's
graphs can be checked against torch's own forward pass and run through W8A8 on rocm."""
import numpy as np

from onnx_writer import Model


def _torch():
    import torch
    return torch


def _np(t) -> np.ndarray:
    return t.detach().cpu().numpy().astype(np.float32)


def _randomize_bn(bn, gen):
    torch = _torch()
    with torch.no_grad():
        bn.weight.copy_(torch.rand(bn.num_features, generator=gen) + 0.5)
        bn.bias.copy_(torch.randn(bn.num_features, generator=gen) * 0.1)
        bn.running_mean.copy_(torch.randn(bn.num_features, generator=gen) * 0.1)
        bn.running_var.copy_(torch.rand(bn.num_features, generator=gen) + 0.5)


class Emitter:
    """Appends the ONNX nodes of torch modules to a Model, in forward order."""

    def __init__(self, m: Model):
        self.m = m

    def conv(self, x: str, c, pads=None) -> str:
        args = [x, self.m.init(_np(c.weight))] + ([self.m.init(_np(c.bias))] if c.bias is not None else [])
        ph, pw = c.padding
        return self.m.node("Conv", args, kernel_shape=list(c.kernel_size), strides=list(c.stride),
                           pads=pads or [ph, pw, ph, pw], dilations=list(c.dilation), group=c.groups)

    def bn(self, x: str, b) -> str:
        return self.m.node("BatchNormalization", [x, self.m.init(_np(b.weight)), self.m.init(_np(b.bias)),
                                                  self.m.init(_np(b.running_mean)), self.m.init(_np(b.running_var))],
                           epsilon=float(b.eps))

    def relu(self, x: str) -> str:
        return self.m.node("Relu", [x])

    def relu6(self, x: str) -> str:
        if self.m.opset < 11:
            return self.m.node("Clip", [x], min=0.0, max=6.0)
        return self.m.node("Clip", [x, self.m.init(np.array(0.0, np.float32)), self.m.init(np.array(6.0, np.float32))])

    def maxpool(self, x: str, k: int, s: int, p: int, ceil: bool = False) -> str:
        return self.m.node("MaxPool", [x], kernel_shape=[k, k], strides=[s, s], pads=[p, p, p, p], ceil_mode=int(ceil))

    def gap_flatten(self, x: str) -> str:
        return self.m.node("Flatten", [self.m.node("GlobalAveragePool", [x])], axis=1)

    def linear(self, x: str, fc) -> str:
        return self.m.node("Gemm", [x, self.m.init(_np(fc.weight)), self.m.init(_np(fc.bias))], transB=1)


def resnet18(batch: int, seed: int = 0, classes: int = 1000):
    """torchvision's ResNet-18 layout in torch (random weights and BN statistics) and its ONNX
    bytes (opset 13, as torch.onnx.export writes it)."""
    torch = _torch()
    nn = torch.nn
    gen = torch.Generator().manual_seed(seed)
    torch.manual_seed(seed)

    class Block(nn.Module):
        def __init__(self, cin, cout, stride):
            super().__init__()
            self.conv1 = nn.Conv2d(cin, cout, 3, stride, 1, bias=False)
            self.bn1 = nn.BatchNorm2d(cout)
            self.conv2 = nn.Conv2d(cout, cout, 3, 1, 1, bias=False)
            self.bn2 = nn.BatchNorm2d(cout)
            self.down = None
            if stride != 1 or cin != cout:
                self.down = nn.Sequential(nn.Conv2d(cin, cout, 1, stride, bias=False), nn.BatchNorm2d(cout))

        def forward(self, x):
            y = torch.relu(self.bn1(self.conv1(x)))
            y = self.bn2(self.conv2(y))
            return torch.relu(y + (self.down(x) if self.down is not None else x))

    class Net(nn.Module):
        def __init__(self):
            super().__init__()
            self.conv1 = nn.Conv2d(3, 64, 7, 2, 3, bias=False)
            self.bn1 = nn.BatchNorm2d(64)
            self.pool = nn.MaxPool2d(3, 2, 1)
            blocks, cin = [], 64
            for stage, c in enumerate((64, 128, 256, 512)):
                for i in range(2):
                    blocks.append(Block(cin, c, 2 if stage > 0 and i == 0 else 1))
                    cin = c
            self.blocks = nn.ModuleList(blocks)
            self.fc = nn.Linear(512, classes)

        def forward(self, x):
            x = self.pool(torch.relu(self.bn1(self.conv1(x))))
            for b in self.blocks:
                x = b(x)
            return self.fc(torch.flatten(nn.functional.adaptive_avg_pool2d(x, 1), 1))

    net = Net().eval()
    for mod in net.modules():
        if isinstance(mod, nn.BatchNorm2d):
            _randomize_bn(mod, gen)
    m = Model(13)
    e = Emitter(m)
    x = m.input("x", (batch, 3, 224, 224))
    h = e.maxpool(e.relu(e.bn(e.conv(x, net.conv1), net.bn1)), 3, 2, 1)
    for b in net.blocks:
        y = e.relu(e.bn(e.conv(h, b.conv1), b.bn1))
        y = e.bn(e.conv(y, b.conv2), b.bn2)
        short = e.bn(e.conv(h, b.down[0]), b.down[1]) if b.down is not None else h
        h = e.relu(m.node("Add", [y, short]))
    out = e.linear(e.gap_flatten(h), net.fc)
    m.output(out, (batch, classes))
    return net, m.bytes()


def edge_net(batch: int, opset: int, seed: int = 1):
    """A small network over the importer's less common forms: Conv bias, dilation, asymmetric
    pads (an explicit pad), a depthwise group, ReLU6 as Clip (attributes before opset 11,
    inputs after), MaxPool with ceil_mode, Dropout / Identity, the Shape-Gather-Unsqueeze-
    Concat-Reshape flatten of older exporters, Gemm with alpha and beta."""
    torch = _torch()
    nn = torch.nn
    gen = torch.Generator().manual_seed(seed)
    torch.manual_seed(seed)
    c1 = nn.Conv2d(3, 16, 3, 1, 0, bias=True)             # run with pads (0, 0, 1, 1): asymmetric
    bn = nn.BatchNorm2d(16)
    dw = nn.Conv2d(16, 16, 3, 1, 2, dilation=2, groups=16, bias=True)
    pw = nn.Conv2d(16, 24, 1, bias=False)
    fc = nn.Linear(24 * 5 * 5, 10)                        # 8x8 pooled 3/2 with pad 1, ceil: 5x5
    _randomize_bn(bn, gen)
    for mod in (c1, bn, dw, pw, fc):
        mod.eval()

    def forward(x):
        y = nn.functional.pad(x, (0, 1, 0, 1))             # (left, right, top, bottom)
        y = torch.clamp(bn(c1(y)), 0.0, 6.0)
        y = torch.clamp(dw(y), 0.0, 6.0)
        y = nn.functional.max_pool2d(pw(y), 3, 2, 1, ceil_mode=True)
        y = torch.flatten(y, 1)
        return 0.5 * (y @ fc.weight.T) + fc.bias          # Gemm alpha 0.5, beta 0.5 on 2 * bias

    m = Model(opset)
    e = Emitter(m)
    x = m.input("x", (batch, 3, 9, 9))
    y = e.relu6(e.bn(e.conv(x, c1, pads=[0, 0, 1, 1]), bn))
    y = e.relu6(e.conv(y, dw))
    y = m.node("Dropout", [m.node("Identity", [e.maxpool(e.conv(y, pw), 3, 2, 1, ceil=True)])])
    shape = m.node("Shape", [y])
    n0 = m.node("Unsqueeze", [m.node("Gather", [shape, m.init(np.array(0, np.int64))], axis=0)], axes=[0]) \
        if opset < 13 else m.node("Unsqueeze", [m.node("Gather", [shape, m.init(np.array(0, np.int64))], axis=0),
                                                 m.init(np.array([0], np.int64))])
    flat = m.node("Reshape", [y, m.node("Concat", [n0, m.init(np.array([-1], np.int64))], axis=0)])
    out = m.node("Gemm", [flat, m.init(_np(fc.weight)), m.init(_np(fc.bias) * 2)], transB=1, alpha=0.5, beta=0.5)
    m.output(out, (batch, 10))
    return forward, m.bytes()


# torchvision's MobileNetV2 stages: (expansion t, output channels c, blocks n, first stride s)
MNV2_STAGES = ((1, 16, 1, 1), (6, 24, 2, 2), (6, 32, 3, 2), (6, 64, 4, 2), (6, 96, 3, 1), (6, 160, 3, 2),
               (6, 320, 1, 1))


def mobilenet_v2(batch: int, seed: int = 0, classes: int = 1000):
    """torchvision's MobileNetV2 layout in torch (random weights and BN statistics): a 3x3/2
    stem, inverted residual blocks (1x1 expansion + BN + ReLU6, 3x3 depthwise + BN + ReLU6,
    1x1 linear projection + BN, the residual add where stride 1 keeps the width), a 1x1 conv to
    1280 channels, global average pooling and the classifier; and its ONNX bytes (opset 13,
    BatchNormalization nodes, ReLU6 as Clip with min/max inputs)."""
    torch = _torch()
    nn = torch.nn
    gen = torch.Generator().manual_seed(seed)
    torch.manual_seed(seed)

    def cbr(cin, cout, k, s, groups=1, relu=True):
        layers = [nn.Conv2d(cin, cout, k, s, (k - 1) // 2, groups=groups, bias=False), nn.BatchNorm2d(cout)]
        return nn.Sequential(*layers, *([nn.ReLU6()] if relu else []))

    class Block(nn.Module):
        def __init__(self, cin, cout, stride, t):
            super().__init__()
            hid = cin * t
            self.res = stride == 1 and cin == cout
            self.layers = nn.Sequential(*([cbr(cin, hid, 1, 1)] if t != 1 else []), cbr(hid, hid, 3, stride, hid),
                                        cbr(hid, cout, 1, 1, relu=False))

        def forward(self, x):
            return x + self.layers(x) if self.res else self.layers(x)

    class Net(nn.Module):
        def __init__(self):
            super().__init__()
            feats, cin = [cbr(3, 32, 3, 2)], 32
            for t, c, n, s in MNV2_STAGES:
                for i in range(n):
                    feats.append(Block(cin, c, s if i == 0 else 1, t))
                    cin = c
            feats.append(cbr(cin, 1280, 1, 1))
            self.features = nn.Sequential(*feats)
            self.fc = nn.Linear(1280, classes)

        def forward(self, x):
            return self.fc(torch.flatten(nn.functional.adaptive_avg_pool2d(self.features(x), 1), 1))

    net = Net().eval()
    for mod in net.modules():
        if isinstance(mod, nn.BatchNorm2d):
            _randomize_bn(mod, gen)
    m = Model(13)
    e = Emitter(m)

    def emit_cbr(x, seq):
        y = e.bn(e.conv(x, seq[0]), seq[1])
        return e.relu6(y) if len(seq) == 3 else y

    h = m.input("x", (batch, 3, 224, 224))
    for f in net.features:
        if isinstance(f, Block):
            y = h
            for seq in f.layers:
                y = emit_cbr(y, seq)
            h = m.node("Add", [h, y]) if f.res else y
        else:
            h = emit_cbr(h, f)
    out = e.linear(e.gap_flatten(h), net.fc)
    m.output(out, (batch, classes))
    return net, m.bytes()
