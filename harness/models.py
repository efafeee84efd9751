"""Float graph builders for the W8A8 benchmark configurations.

Each builder returns an unoptimized float32 graph with constant weights, laid
out as MIRA's front ends produce it, so lowering (harness.lowering.prepare,
then w8a8) gives the op and epilogue structure MIRA's compiler gives it:

* dense layers are `matmul` + `add(bias)` (+ activation), as in
  examples/mlp.mira (`x @ w + b`);
* convolutions with folded batch norm are `conv2d` + `add(bias [O,1,1])`,
  ReLU is `relu`, ReLU6 is `maximum(0)` then `minimum(6)` with 0-d constants
  (how mira/frontends/onnx_import.py:477-485 imports Clip);
* max pooling with padding is `pad(-inf)` + `maxpool2d`
  (mira/frontends/onnx_import.py:391-395), global average pooling is
  `reduce_mean(axes=(2, 3), keepdims)` (:416-420), flatten is `reshape`.

Weights are drawn from one seeded generator in a fixed order; the same
(seed, architecture) at any batch size gives the same weights, so a
small-batch twin can be used for calibration.
"""
from __future__ import annotations

import numpy as np

from .graph import Graph, conv_out


def _normal(rng, shape, std):
    return (rng.standard_normal(shape) * std).astype(np.float32)


def mira_random_weight(rng, shape, dtype=np.float32) -> np.ndarray:
    """The seeded weights MIRA's elaborator gives a const parameter (mira/elaborate.py:1114-1123),
    drawn in parameter order from one generator: rank 1 -> 1 + 0.1 N; rank 4 -> N / sqrt(C*KH*KW);
    any other rank -> N / sqrt(shape[-2]); each draw rounded once, from f64 to `dtype`."""
    if len(shape) == 0:
        return np.array(rng.standard_normal(), dtype=dtype)
    if len(shape) == 1:
        return (1.0 + 0.1 * rng.standard_normal(shape)).astype(dtype)
    fan_in = int(np.prod(shape[1:])) if len(shape) == 4 else shape[-2]
    return (rng.standard_normal(shape) / np.sqrt(fan_in)).astype(dtype)


# ---------------------------------------------------------------- MLPs

def mlp_dense(batch: int = 256, k: int = 64, n: int = 10, seed: int = 0) -> Graph:
    """x f32[batch, k] @ w f32[k, n] ~ N(0, 0.1) + b zeros (a zero bias is removed by simplify)."""
    rng = np.random.default_rng(seed)
    g = Graph("mlp_dense")
    x = g.input("x", (batch, k))
    w = g.const(_normal(rng, (k, n), 0.1))
    b = g.const(np.zeros(n, np.float32))
    g.outputs = [g.op("add", [g.op("matmul", [x, w]), b])]
    return g


def mlp_mira(batch: int = 64, seed: int = 0) -> Graph:
    """examples/mlp.mira: 784 -> 512 -> 256 -> 10 with ReLU, then softmax(axis=1)."""
    rng = np.random.default_rng(seed)
    g = Graph("mlp")
    h = g.input("x", (batch, 784))
    dims = [(784, 512), (512, 256), (256, 10)]
    params = [(mira_random_weight(rng, d), mira_random_weight(rng, (d[1],))) for d in dims]
    for i, (w, b) in enumerate(params):
        h = g.op("add", [g.op("matmul", [h, g.const(w)]), g.const(b)])
        if i < 2:
            h = g.op("relu", [h])
    g.outputs = [g.op("softmax", [h], {"axis": 1})]
    return g


def mlp_50m(batch: int = 4096, seed: int = 0) -> Graph:
    """4 dense layers 4096->4096 (x3) and 4096->1000, ReLU between, W ~ N(0, 1/sqrt(4096)),
    biases ~ N(0, 0.1): 54.4 M parameters."""
    rng = np.random.default_rng(seed)
    g = Graph("mlp50m")
    h = g.input("x", (batch, 4096))
    dims = [(4096, 4096)] * 3 + [(4096, 1000)]
    for i, (k, n) in enumerate(dims):
        w = g.const(_normal(rng, (k, n), 1.0 / np.sqrt(4096)))
        b = g.const(_normal(rng, (n,), 0.1))
        h = g.op("add", [g.op("matmul", [h, w]), b])
        if i < len(dims) - 1:
            h = g.op("relu", [h])
    g.outputs = [h]
    return g


# ---------------------------------------------------------------- CNNs

class _ConvNet:
    """Helper that draws conv+BN parameters in a fixed order.  bn_epilogue=False folds BN
    into the weights and a bias; bn_epilogue=True keeps it as the `mul` + `add` of
    per-channel constants that MIRA's ONNX importer emits for BatchNormalization
    (mira/frontends/onnx_import.py:423-431), after a bias-free conv."""

    def __init__(self, g: Graph, seed: int, bn_epilogue: bool = False):
        self.g = g
        self.rng = np.random.default_rng(seed)
        self.bn_epilogue = bn_epilogue

    def conv(self, x, o: int, k: int, stride: int = 1, pad: int = 0, groups: int = 1, bn: bool = True):
        """conv2d + folded BatchNorm: Kaiming-normal (fan_out) weights scaled by gamma/sqrt(var+eps),
        bias beta - mean*gamma/sqrt(var+eps), with random BN statistics so the bias is not zero."""
        rng = self.rng
        c = x.type.shape[1]
        w = _normal(rng, (o, c // groups, k, k), np.sqrt(2.0 / (o * k * k / groups)))
        attrs = {"stride": (stride, stride), "padding": (pad, pad)}
        if groups != 1:
            attrs["groups"] = groups
        if bn:
            gamma = rng.uniform(0.5, 1.5, o)
            beta = rng.normal(0.0, 0.1, o)
            mean = rng.normal(0.0, 0.1, o)
            var = rng.uniform(0.5, 1.5, o)
            s = gamma / np.sqrt(var + 1e-5)
            if self.bn_epilogue:
                y = self.g.op("conv2d", [x, self.g.const(w)], attrs)
                y = self.g.op("mul", [y, self.g.const(s.reshape(o, 1, 1).astype(np.float32))])
                return self.g.op("add", [y, self.g.const((beta - mean * s).reshape(o, 1, 1).astype(np.float32))])
            w = (w * s.reshape(-1, 1, 1, 1)).astype(np.float32)
            bias = (beta - mean * s).astype(np.float32)
        else:
            bias = np.zeros(o, np.float32)
        y = self.g.op("conv2d", [x, self.g.const(w)], attrs)
        return self.g.op("add", [y, self.g.const(bias.reshape(o, 1, 1))])

    def relu(self, x):
        return self.g.op("relu", [x])

    def relu6(self, x):
        g = self.g
        y = g.op("maximum", [x, g.const(np.array(0.0, np.float32))])
        return g.op("minimum", [y, g.const(np.array(6.0, np.float32))])

    def head(self, x, classes: int):
        """Global average pool, flatten, fully connected."""
        g = self.g
        n, c = x.type.shape[:2]
        pooled = g.op("reduce_mean", [x], {"axes": (2, 3), "keepdims": True})
        flat = g.op("reshape", [pooled], {"shape": (n, c)})
        w = _normal(self.rng, (c, classes), 1.0 / np.sqrt(c))
        b = _normal(self.rng, (classes,), 0.01)
        return g.op("add", [g.op("matmul", [flat, g.const(w)]), g.const(b)])


def resnet18(batch: int = 256, seed: int = 0, classes: int = 1000, bn_epilogue: bool = False) -> Graph:
    """torchvision ResNet-18: 7x7/2 stem, 3x3/2 max pool, 4 stages of two basic blocks (64, 128,
    256, 512 channels; stride-2 1x1 downsample convs), GAP, fc.  BN folded, or (bn_epilogue)
    as the ONNX importer's per-channel mul + add."""
    g = Graph("resnet18")
    net = _ConvNet(g, seed, bn_epilogue)
    x = g.input("x", (batch, 3, 224, 224))
    h = net.relu(net.conv(x, 64, 7, 2, 3))
    h = g.op("pad", [h], {"pads": ((0, 0), (0, 0), (1, 1), (1, 1)), "value": -np.inf})
    h = g.op("maxpool2d", [h], {"size": 3, "stride": 2})
    c_in = 64
    for stage, c in enumerate((64, 128, 256, 512)):
        for blk in range(2):
            stride = 2 if stage > 0 and blk == 0 else 1
            y = net.relu(net.conv(h, c, 3, stride, 1))
            y = net.conv(y, c, 3, 1, 1)
            shortcut = net.conv(h, c, 1, stride, 0) if (stride != 1 or c_in != c) else h
            h = net.relu(g.op("add", [y, shortcut]))
            c_in = c
    g.outputs = [net.head(h, classes)]
    return g


def mobilenet_v2(batch: int = 128, seed: int = 0, classes: int = 1000, bn_epilogue: bool = False) -> Graph:
    """torchvision MobileNetV2: 3x3/2 stem, 17 inverted residual blocks (1x1 expand + ReLU6,
    3x3 depthwise + ReLU6, 1x1 linear projection, residual when shapes allow), 1x1 conv to
    1280 + ReLU6, GAP, fc.  BN folded, or (bn_epilogue) as the ONNX importer's mul + add."""
    g = Graph("mobilenet_v2")
    net = _ConvNet(g, seed, bn_epilogue)
    x = g.input("x", (batch, 3, 224, 224))
    h = net.relu6(net.conv(x, 32, 3, 2, 1))
    c_in = 32
    for t, c, n, s in ((1, 16, 1, 1), (6, 24, 2, 2), (6, 32, 3, 2), (6, 64, 4, 2), (6, 96, 3, 1), (6, 160, 3, 2),
                       (6, 320, 1, 1)):
        for i in range(n):
            stride = s if i == 0 else 1
            hidden = c_in * t
            y = h
            if t != 1:
                y = net.relu6(net.conv(y, hidden, 1))
            y = net.relu6(net.conv(y, hidden, 3, stride, 1, groups=hidden))
            y = net.conv(y, c, 1)
            h = g.op("add", [y, h]) if (stride == 1 and c_in == c) else y
            c_in = c
    h = net.relu6(net.conv(h, 1280, 1))
    g.outputs = [net.head(h, classes)]
    return g


def cnn_mira(batch: int = 16, seed: int = 0) -> Graph:
    """examples/cnn.mira: two conv(3x3, pad 1) + bias + relu + maxpool(2) blocks, flatten, dense, softmax."""
    rng = np.random.default_rng(seed)
    g = Graph("cnn")
    h = g.input("img", (batch, 1, 28, 28))
    params = [(mira_random_weight(rng, (o, c, 3, 3)), mira_random_weight(rng, (o, 1, 1))) for o, c in ((16, 1), (32, 16))]
    wf = mira_random_weight(rng, (1568, 10))
    bf = mira_random_weight(rng, (10,))
    for k, b in params:
        y = g.op("conv2d", [h, g.const(k)], {"stride": (1, 1), "padding": (1, 1)})
        y = g.op("relu", [g.op("add", [y, g.const(b)])])
        h = g.op("maxpool2d", [y], {"size": 2, "stride": 2})
    flat = g.op("reshape", [h], {"shape": (batch, h.type.numel // batch)})
    g.outputs = [g.op("softmax", [g.op("add", [g.op("matmul", [flat, g.const(wf)]), g.const(bf)])],
                       {"axis": -1})]
    return g


BUILDERS = {
    "mlp_dense": mlp_dense,
    "mlp": mlp_mira,
    "cnn": cnn_mira,
    "mlp50m": mlp_50m,
    "resnet18": resnet18,
    "mobilenet_v2": mobilenet_v2,
}


def image_batch(shape, seed: int) -> np.ndarray:
    """Synthetic images ~ U(0, 1)."""
    return np.random.default_rng(seed).uniform(0.0, 1.0, shape).astype(np.float32)


def normal_batch(shape, seed: int) -> np.ndarray:
    return np.random.default_rng(seed).standard_normal(shape).astype(np.float32)


def conv_macs(g: Graph) -> int:
    """Multiply-accumulates of every int8 contraction (qconv2d/qmatmul) in a quantized graph."""
    total = 0
    for op in g.ops:
        if op.kind == "qconv2d":
            n, o, oh, ow = op.result.type.shape
            _, c, kh, kw = op.attrs["q"].shape
            total += n * o * oh * ow * c * kh * kw
        elif op.kind == "qmatmul":
            k, n = op.attrs["q"].shape
            total += (op.result.type.numel // n) * n * k
    return total


__all__ = ["BUILDERS", "conv_out", "conv_macs"]


# ---------------------------------------------------------------- character-level GPT, one decode step

class GPTConfig:
    """The decode configuration of the character-level GPT of examples/gpt_text.mira (with the
    widths of examples/gpt_text_train.py:30): L layers of width D with H heads, MLP width F,
    vocabulary V, and a KV cache of T positions (prompt + generated tokens)."""

    def __init__(self, L: int = 2, D: int = 64, H: int = 4, F: int = 128, V: int = 65, T: int = 272):
        self.L, self.D, self.H, self.F, self.V, self.T = L, D, H, F, V, T


def gpt_params(cfg: GPTConfig, seed: int = 0) -> dict:
    """Random weights with the distribution of mira/elaborate.py:1114-1123 (as `generate`'s
    const parameters would get): embedding and position tables, per-layer projections and
    layernorm gains/biases, final layernorm and output projection."""
    rng = np.random.default_rng(seed)
    D, F, V, T = cfg.D, cfg.F, cfg.V, cfg.T
    p = {"emb": mira_random_weight(rng, (V, D)), "pos": mira_random_weight(rng, (T, D))}
    for l in range(cfg.L):
        for name, shape in (("wq", (D, D)), ("wk", (D, D)), ("wv", (D, D)), ("wo", (D, D)), ("w1", (D, F)),
                            ("w2", (F, D)), ("g1", (D,)), ("b1", (D,)), ("g2", (D,)), ("b2", (D,))):
            p[f"{name}{l}"] = mira_random_weight(rng, shape)
    p["gf"], p["bf"] = mira_random_weight(rng, (D,)), mira_random_weight(rng, (D,))
    p["wout"] = mira_random_weight(rng, (D, V))
    return p


def gpt_decode_step(cfg: GPTConfig, batch: int, params: dict) -> Graph:
    """One decode step of `generate` (examples/gpt_text.mira, the while-loop body) as a graph
    without control flow, so W8A8 can quantize it (mira/quantize.py:84-85 refuses control flow).

    Inputs:  h     f32[B, D]        token embedding + position embedding of the current token
             mask  f32[1,1,1,T+1]   0 for cache rows already written and for the current token,
                                    -10000 elsewhere (the `(seen - 1) * 10000` of the reference)
             kc{l}, vc{l} f32[B, T, D]  the layer's key/value cache
    Outputs: logits f32[B, V], then k{l}, v{l} f32[B, D] for the host to write at the position.
    The current token's key/value join the cache by concatenation (slot T), so the graph keeps
    static shapes at every position."""
    L, D, H, V, T = cfg.L, cfg.D, cfg.H, cfg.V, cfg.T
    hd = D // H
    g = Graph("gpt_step")
    h = g.input("h", (batch, D))
    mask = g.input("mask", (1, 1, 1, T + 1))
    caches = [(g.input(f"kc{l}", (batch, T, D)), g.input(f"vc{l}", (batch, T, D))) for l in range(L)]
    c = lambda name: g.const(params[name])
    scale = g.const(np.float32(1.0 / np.sqrt(hd)))
    kv_out = []
    for l in range(L):
        kc, vc = caches[l]
        x = g.op("layernorm", [h, c(f"g1{l}"), c(f"b1{l}")], {"eps": 1e-5})
        q = g.op("matmul", [x, c(f"wq{l}")])
        k = g.op("matmul", [x, c(f"wk{l}")])
        v = g.op("matmul", [x, c(f"wv{l}")])
        kv_out += [k, v]
        q4 = g.op("transpose", [g.op("reshape", [q], {"shape": (batch, 1, H, hd)})], {"perm": (0, 2, 1, 3)})
        keys = g.op("concat", [kc, g.op("reshape", [k], {"shape": (batch, 1, D)})], {"axis": 1})
        vals = g.op("concat", [vc, g.op("reshape", [v], {"shape": (batch, 1, D)})], {"axis": 1})
        k4 = g.op("transpose", [g.op("reshape", [keys], {"shape": (batch, T + 1, H, hd)})], {"perm": (0, 2, 3, 1)})
        v4 = g.op("transpose", [g.op("reshape", [vals], {"shape": (batch, T + 1, H, hd)})], {"perm": (0, 2, 1, 3)})
        s = g.op("add", [g.op("mul", [g.op("matmul", [q4, k4]), scale]), mask])
        o4 = g.op("matmul", [g.op("softmax", [s], {"axis": -1}), v4])
        o = g.op("reshape", [g.op("transpose", [o4], {"perm": (0, 2, 1, 3)})], {"shape": (batch, D)})
        h = g.op("add", [h, g.op("matmul", [o, c(f"wo{l}")])])
        y = g.op("layernorm", [h, c(f"g2{l}"), c(f"b2{l}")], {"eps": 1e-5})
        h = g.op("add", [h, g.op("matmul", [g.op("gelu", [g.op("matmul", [y, c(f"w1{l}")])]), c(f"w2{l}")])])
    logits = g.op("matmul", [g.op("layernorm", [h, c("gf"), c("bf")], {"eps": 1e-5}), c("wout")])
    g.outputs = [logits] + kv_out
    return g


def gpt_step_feeds(cfg: GPTConfig, params: dict, tokens: np.ndarray, t: int, caches: list) -> dict:
    """Host side of one decode step at position t: embedding gather, position row, cache mask."""
    h = (params["emb"][tokens[:, t]] + params["pos"][t]).astype(np.float32)
    mask = np.full((1, 1, 1, cfg.T + 1), -10000.0, np.float32)
    mask[..., :t] = 0.0
    mask[..., cfg.T] = 0.0
    feeds = {"h": h, "mask": mask}
    for l, (kc, vc) in enumerate(caches):
        feeds[f"kc{l}"], feeds[f"vc{l}"] = kc, vc
    return feeds


def gpt_decode(run, cfg: GPTConfig, params: dict, prompt: np.ndarray, new_tokens: int):
    """Greedy decoding as `generate` does it (keep the prompt, then argmax), with `run(feeds) ->
    [logits, k0, v0, ...]` executing one decode step.  Returns tokens [B, P + new_tokens] and the
    logits of every step."""
    B, P = prompt.shape
    total = P + new_tokens
    assert total <= cfg.T
    tokens = np.zeros((B, total), np.int32)
    tokens[:, :P] = prompt
    caches = [(np.zeros((B, cfg.T, cfg.D), np.float32), np.zeros((B, cfg.T, cfg.D), np.float32))
              for _ in range(cfg.L)]
    all_logits = []
    for t in range(total - 1):
        out = run(gpt_step_feeds(cfg, params, tokens, t, caches))
        logits = out[0]
        all_logits.append(logits)
        for l in range(cfg.L):
            caches[l][0][:, t] = out[1 + 2 * l]
            caches[l][1][:, t] = out[2 + 2 * l]
        if t + 1 >= P:
            tokens[:, t + 1] = np.argmax(logits, axis=1)
    return tokens, all_logits
