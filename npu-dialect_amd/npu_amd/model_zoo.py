"""Whole networks as linalg text, in the form of the reference's model zoo.

The reference keeps ~100 networks as MLIR text under test/models/, written by
its generator (tools/gen_model_mlir.py): NCHW f16 tensors, every layer a
`linalg.conv_2d_nchw_fchw` (pooling written as a stride-2 3x3 conv, the
classifier as a conv over the last feature map) or a `linalg.matmul`, each
fed by a `linalg.fill` of zero, a `tensor.pad` of zeros before it when it
pads, and `linalg.generic` ReLU (`arith.maximumf` with 0) and residual-add
(`arith.addf`) epilogues.  The GPU box has no reference checkout, so the
networks it runs are written here, op for op in that form; a CPU test checks
each against the reference's file (ops, dataflow, types, maps, bodies, pads,
strides).

Families: ResNet with basic or bottleneck blocks (resnet18, resnet34,
resnet50, resnet_deep_20), VGG, sequential CNNs (srcnn, espcn), the GAN
generator (dcgan_generator) and the fully connected autoencoders.
"""
from __future__ import annotations


def _t(shape, elem="f16"):
    return "tensor<" + "x".join(str(d) for d in shape) + "x" + elem + ">"


class _Net:
    """Accumulates one function's text: parameters, then ops, each value
    named by a prefix and a running number."""

    def __init__(self, elem="f16"):
        self.elem = elem
        self.params = []
        self.lines = []
        self.n = 0

    def name(self, prefix):
        v = f"%{prefix}{self.n}"
        self.n += 1
        return v

    def param(self, name, shape):
        self.params.append((name, shape))
        return name

    def pad(self, x, shape, p):
        e = self.elem
        out = [shape[0], shape[1], shape[2] + 2 * p, shape[3] + 2 * p]
        v = self.name("pad")
        self.lines += [f"{v} = tensor.pad {x} low[0, 0, {p}, {p}] high[0, 0, {p}, {p}] {{",
                       "^bb0(%a0: index, %a1: index, %a2: index, %a3: index):",
                       f"  tensor.yield %cst : {e}",
                       f"}} : {_t(shape, e)} to {_t(out, e)}"]
        return v, out

    def conv(self, x, xshape, w, wshape, stride):
        e = self.elem
        n, _, h, wd = xshape
        f, _, kh, kw = wshape
        out = [n, f, (h - kh) // stride + 1, (wd - kw) // stride + 1]
        init, fill, v = self.name("init"), self.name("fill"), self.name("conv")
        self.lines += [f"{init} = tensor.empty() : {_t(out, e)}",
                       f"{fill} = linalg.fill ins(%cst : {e}) outs({init} : {_t(out, e)}) -> "
                       f"{_t(out, e)}",
                       f"{v} = linalg.conv_2d_nchw_fchw {{",
                       "  dilations = dense<1> : tensor<2xi64>,",
                       f"  strides = dense<{stride}> : tensor<2xi64>",
                       f"}} ins({x}, {w} : {_t(xshape, e)}, {_t(wshape, e)})",
                       f"  outs({fill} : {_t(out, e)}) -> {_t(out, e)}"]
        return v, out

    def matmul(self, a, ashape, b, bshape):
        e = self.elem
        out = [ashape[0], bshape[1]]
        init, fill, v = self.name("init"), self.name("fill"), self.name("mm")
        self.lines += [f"{init} = tensor.empty() : {_t(out, e)}",
                       f"{fill} = linalg.fill ins(%cst : {e}) outs({init} : {_t(out, e)}) -> "
                       f"{_t(out, e)}",
                       f"{v} = linalg.matmul ins({a}, {b} : {_t(ashape, e)}, {_t(bshape, e)})",
                       f"  outs({fill} : {_t(out, e)}) -> {_t(out, e)}"]
        return v, out

    def _eltwise(self, ins, shape, prefix, body):
        e = self.elem
        rank = len(shape)
        ids = ", ".join(f"d{i}" for i in range(rank))
        amap = f"affine_map<({ids}) -> ({ids})>"
        empty, v = self.name("empty"), self.name(prefix)
        names = ["in"] if len(ins) == 1 else ["a", "b"]
        args = ", ".join([f"%{a}: {e}" for a in names] + [f"%out: {e}"])
        maps = ", ".join([amap] * (len(ins) + 1))
        its = ", ".join(['"parallel"'] * rank)
        self.lines += [f"{empty} = tensor.empty() : {_t(shape, e)}",
                       f"{v} = linalg.generic {{",
                       f"  indexing_maps = [{maps}],",
                       f"  iterator_types = [{its}]",
                       f"}} ins({', '.join(ins)} : {', '.join([_t(shape, e)] * len(ins))})",
                       f"  outs({empty} : {_t(shape, e)}) {{",
                       f"^bb0({args}):"] + [f"  {b}" for b in body] + [f"}} -> {_t(shape, e)}"]
        return v

    def relu(self, x, shape):
        e = self.elem
        return self._eltwise([x], shape, "relu", [f"%z = arith.constant 0.0 : {e}",
                                                  f"%m = arith.maximumf %in, %z : {e}",
                                                  f"linalg.yield %m : {e}"])

    def add(self, a, b, shape):
        e = self.elem
        return self._eltwise([a, b], shape, "add", [f"%sum = arith.addf %a, %b : {e}",
                                                    f"linalg.yield %sum : {e}"])

    def conv_block(self, x, shape, w, cout, k, stride, pad, relu=True):
        """[pad] -> conv [-> ReLU]; the filter parameter is declared by the caller."""
        if pad:
            x, shape = self.pad(x, shape, pad)
        v, out = self.conv(x, shape, w, [cout, shape[1], k, k], stride)
        if relu:
            v = self.relu(v, out)
        return v, out

    def text(self, fname, result, rshape):
        params = ",\n    ".join(f"{n}: {_t(s, self.elem)}" for n, s in self.params)
        body = "\n".join("  " + ln for ln in self.lines)
        return (f"func.func @{fname}(\n    {params}) -> {_t(rshape, self.elem)} {{\n"
                f"  %cst = arith.constant 0.0 : {self.elem}\n{body}\n"
                f"  return {result} : {_t(rshape, self.elem)}\n}}\n")


def resnet(layers, block="basic", classes=1000, elem="f16"):
    """ResNet on 1x3x224x224: 7x7/2 stem, a stride-2 3x3 conv standing for
    the max pool, four stages of basic (3x3, 3x3) or bottleneck (1x1, 3x3,
    1x1, 4x expansion) blocks with a 1x1 shortcut conv where the shape
    changes (stride 2 at each stage's first block after the first stage),
    and the classifier as a 7x7 conv."""
    net = _Net(elem)
    chans = [64, 128, 256, 512]
    outs = [c * 4 for c in chans] if block == "bottleneck" else list(chans)
    net.param("%input", [1, 3, 224, 224])
    net.param("%w_conv1", [64, 3, 7, 7])
    net.param("%w_pool", [64, 64, 3, 3])
    plan = []
    for si in range(4):
        oc = outs[si]
        first_in = outs[si - 1] if si else 64
        for bi in range(layers[si]):
            ic = first_in if bi == 0 else oc
            st = 2 if si and bi == 0 else 1
            pre = f"%w_s{si}_b{bi}"
            if block == "basic":
                net.param(f"{pre}_c1", [oc, ic, 3, 3])
                net.param(f"{pre}_c2", [oc, oc, 3, 3])
            else:
                mid = oc // 4
                net.param(f"{pre}_c1", [mid, ic, 1, 1])
                net.param(f"{pre}_c2", [mid, mid, 3, 3])
                net.param(f"{pre}_c3", [oc, mid, 1, 1])
            sc = ic != oc or st > 1
            if sc:
                net.param(f"{pre}_sc", [oc, ic, 1, 1])
            plan.append((pre, ic, oc, st, sc))
    net.param("%w_fc", [classes, outs[3], 7, 7])

    x, shape = net.conv_block("%input", [1, 3, 224, 224], "%w_conv1", 64, 7, 2, 3)
    x, shape = net.conv_block(x, shape, "%w_pool", 64, 3, 2, 1)
    for pre, ic, oc, st, sc in plan:
        inp, ishape = x, shape
        if block == "basic":
            y, ys = net.conv_block(inp, ishape, f"{pre}_c1", oc, 3, st, 1)
            y, ys = net.conv_block(y, ys, f"{pre}_c2", oc, 3, 1, 1, relu=False)
        else:
            mid = oc // 4
            y, ys = net.conv_block(inp, ishape, f"{pre}_c1", mid, 1, 1, 0)
            y, ys = net.conv_block(y, ys, f"{pre}_c2", mid, 3, st, 1)
            y, ys = net.conv_block(y, ys, f"{pre}_c3", oc, 1, 1, 0, relu=False)
        r = inp
        if sc:
            r, _ = net.conv(inp, ishape, f"{pre}_sc", [oc, ic, 1, 1], st)
        a = net.add(y, r, ys)
        x, shape = net.relu(a, ys), ys
    v, out = net.conv(x, shape, "%w_fc", [classes, shape[1], shape[2], shape[3]], 1)
    return net.text(f"resnet_{block}_{'_'.join(str(n) for n in layers)}", v, out)


def vgg(cfg, name, classes=1000, elem="f16"):
    """VGG on 1x3x224x224: blocks of 3x3 conv + ReLU, each closed by a
    stride-2 3x3 conv standing for the pool, then the classifier as a 7x7
    conv + ReLU and two 1x1 convs (ReLU after the first)."""
    net = _Net(elem)
    net.param("%input", [1, 3, 224, 224])
    c = 3
    for bi, (nconv, ch) in enumerate(cfg):
        for ci in range(nconv):
            net.param(f"%w_b{bi}_c{ci}", [ch, c if ci == 0 else ch, 3, 3])
            c = ch
        net.param(f"%w_b{bi}_pool", [ch, ch, 3, 3])
    net.param("%w_fc1", [4096, c, 7, 7])
    net.param("%w_fc2", [4096, 4096, 1, 1])
    net.param("%w_fc3", [classes, 4096, 1, 1])
    x, shape = "%input", [1, 3, 224, 224]
    for bi, (nconv, ch) in enumerate(cfg):
        for ci in range(nconv):
            x, shape = net.conv_block(x, shape, f"%w_b{bi}_c{ci}", ch, 3, 1, 1)
        x, shape = net.conv_block(x, shape, f"%w_b{bi}_pool", ch, 3, 2, 1)
    v, shape = net.conv(x, shape, "%w_fc1", [4096, shape[1], shape[2], shape[3]], 1)
    x = net.relu(v, shape)
    x, shape = net.conv_block(x, shape, "%w_fc2", 4096, 1, 1, 0)
    x, shape = net.conv_block(x, shape, "%w_fc3", classes, 1, 1, 0, relu=False)
    return net.text(name, x, shape)


def sequential_cnn(specs, name, cin=3, h=224, w=224, classes=1000, elem="f16"):
    """A plain stack of (out channels, kernel, stride, pad, ReLU) conv layers,
    then a 1x1 conv classifier without ReLU (srcnn, espcn)."""
    net = _Net(elem)
    net.param("%input", [1, cin, h, w])
    c = cin
    for i, (oc, k, _, _, _) in enumerate(specs):
        net.param(f"%w{i}", [oc, c, k, k])
        c = oc
    net.param("%w_fc", [classes, c, 1, 1])
    x, shape = "%input", [1, cin, h, w]
    for i, (oc, k, s, p, relu) in enumerate(specs):
        x, shape = net.conv_block(x, shape, f"%w{i}", oc, k, s, p, relu)
    x, shape = net.conv_block(x, shape, "%w_fc", classes, 1, 1, 0, relu=False)
    return net.text(name, x, shape)


def gan_generator(specs, name, cin=100, h=4, w=4, elem="f16"):
    """The generator stack: (out channels, kernel, stride, pad, ReLU) layers
    and nothing after them (dcgan_generator)."""
    net = _Net(elem)
    net.param("%input", [1, cin, h, w])
    c = cin
    for i, (oc, k, _, _, _) in enumerate(specs):
        net.param(f"%w{i}", [oc, c, k, k])
        c = oc
    x, shape = "%input", [1, cin, h, w]
    for i, (oc, k, s, p, relu) in enumerate(specs):
        x, shape = net.conv_block(x, shape, f"%w{i}", oc, k, s, p, relu)
    return net.text(name, x, shape)


def autoencoder(sizes, name, din=784, elem="f16"):
    """Fully connected encoder (matmul + ReLU per size) and the mirrored
    decoder, its last layer without ReLU."""
    net = _Net(elem)
    net.param("%input", [1, din])
    dec = list(reversed(sizes[:-1])) + [din]
    prev = din
    for i, s in enumerate(sizes):
        net.param(f"%w_enc{i}", [prev, s])
        prev = s
    for i, s in enumerate(dec):
        net.param(f"%w_dec{i}", [prev, s])
        prev = s
    x, shape = "%input", [1, din]
    for i, s in enumerate(sizes):
        v, shape = net.matmul(x, shape, f"%w_enc{i}", [shape[1], s])
        x = net.relu(v, shape)
    for i, s in enumerate(dec):
        v, shape = net.matmul(x, shape, f"%w_dec{i}", [shape[1], s])
        x = net.relu(v, shape) if i + 1 < len(dec) else v
    return net.text(name, x, shape)


# Networks by the reference's file name (test/models/<name>.mlir).
MODELS = {
    "resnet18": lambda: resnet([2, 2, 2, 2]),
    "resnet34": lambda: resnet([3, 4, 6, 3]),
    "resnet50": lambda: resnet([3, 4, 6, 3], "bottleneck"),
    "resnet_deep_20": lambda: resnet([3, 3, 3, 3]),
    "vgg11": lambda: vgg([(1, 64), (1, 128), (2, 256), (2, 512), (2, 512)], "vgg11"),
    "srcnn": lambda: sequential_cnn([(64, 9, 1, 4, True), (32, 1, 1, 0, True),
                                     (3, 5, 1, 2, False)], "srcnn", classes=3),
    "espcn": lambda: sequential_cnn([(64, 5, 1, 2, True), (32, 3, 1, 1, True),
                                     (12, 3, 1, 1, False)], "espcn", classes=12),
    "dcgan_generator": lambda: gan_generator([(512, 3, 1, 1, True), (256, 3, 1, 1, True),
                                              (128, 3, 1, 1, True), (64, 3, 1, 1, True),
                                              (3, 3, 1, 1, False)], "dcgan_generator"),
    "autoencoder": lambda: autoencoder([512, 256, 128, 64], "autoencoder"),
    "autoencoder_deep": lambda: autoencoder([1024, 512, 256, 128, 64, 32], "autoencoder_deep",
                                            din=1024),
}


def model(name: str) -> str:
    """The text of test/models/<name>.mlir's network."""
    return MODELS[name]()
