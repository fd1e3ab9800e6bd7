"""The model-level BASELINE configurations as runnable workloads (bench and tests).

* :func:`resnet18` / :func:`resnet18_fuse_groups` -- configuration 5's network: a ResNet-18
  of Lucid's float modules (Conv2d / BatchNorm2d / ReLU, residual adds on
  ``nnq.FloatFunctional``, stubs at both ends) whose static-PTQ flow (fuse -> prepare ->
  calibrate -> convert) yields the quantized module tree the bench times.
* :func:`decoder` -- configuration 4's float decoder (6 layers, d 512, 8 heads, FFN 2048,
  vocab 32000): the Linears as a module tree for ``quantize_dynamic``, the embeddings as
  float32 arrays.
* :class:`Int8Decoder` -- that decoder, after ``quantize_dynamic``, run on the device through
  the C ABI on preallocated buffers, so a whole prefill or decode step is one captured HIP
  graph (positions live in a device counter; the next token comes from an on-device argmax).
  Each Linear is the dynamic module's own forward (:class:`DynLinear`): observer -> qparams
  -> quantize -> W8A8 GEMM on the module's weight operands, bit for bit the same launches as
  ``nnqd.Linear.forward``; the float glue is ``lq_glue.hip``.

Random initialisation only: there is no network in this environment for checkpoints.
"""

from __future__ import annotations

import ctypes

import numpy as np

from lucid_amd import _C
from lucid_amd._tensor import empty, tensor

D_MODEL, HEADS, FFN, VOCAB, LAYERS = 512, 8, 2048, 32000, 6
BATCH, PREFILL, DECODE = 8, 512, 128


def _host(a):
    return tensor(np.asarray(a, np.float32))


# --------------------------------------------------------------------- configuration 5


def resnet18(rng: np.random.Generator, num_classes: int = 1000):
    """ResNet-18 for 3 x 224 x 224 inputs, random BatchNorm statistics and affine terms."""
    import lucid_amd.nn as nn
    import lucid_amd.nn.quantized as nnq

    def bn(c):
        m = nn.BatchNorm2d(c)
        m.running_mean = _host(rng.normal(0, 0.1, c))
        m.running_var = _host(rng.uniform(0.5, 1.5, c))
        m.weight = nn.Parameter(_host(rng.normal(1, 0.1, c)))
        m.bias = nn.Parameter(_host(rng.normal(0, 0.1, c)))
        return m

    class BasicBlock(nn.Module):
        def __init__(self, cin, cout, stride):
            super().__init__()
            self.conv1 = nn.Conv2d(cin, cout, 3, stride=stride, padding=1, bias=False)
            self.bn1 = bn(cout)
            self.relu = nn.ReLU()
            self.conv2 = nn.Conv2d(cout, cout, 3, padding=1, bias=False)
            self.bn2 = bn(cout)
            self.downsample = (nn.Sequential(nn.Conv2d(cin, cout, 1, stride=stride, bias=False), bn(cout))
                               if stride != 1 or cin != cout else None)
            self.skip = nnq.FloatFunctional()

        def forward(self, x):
            out = self.relu(self.bn1(self.conv1(x)))
            out = self.bn2(self.conv2(out))
            identity = self.downsample(x) if self.downsample is not None else x
            return self.skip.add_relu(out, identity)

    class ResNet18(nn.Module):
        def __init__(self):
            super().__init__()
            self.quant = nnq.QuantStub()
            self.conv1 = nn.Conv2d(3, 64, 7, stride=2, padding=3, bias=False)
            self.bn1 = bn(64)
            self.relu = nn.ReLU()
            self.maxpool = nn.MaxPool2d(3, 2, 1)
            chans = [(64, 64, 1), (64, 128, 2), (128, 256, 2), (256, 512, 2)]
            for i, (cin, cout, st) in enumerate(chans, 1):
                setattr(self, f"layer{i}", nn.Sequential(BasicBlock(cin, cout, st), BasicBlock(cout, cout, 1)))
            self.avgpool = nn.AdaptiveAvgPool2d(1)
            self.flatten = nn.Flatten()
            self.fc = nn.Linear(512, num_classes)
            self.dequant = nnq.DeQuantStub()

        def forward(self, x):
            x = self.maxpool(self.relu(self.bn1(self.conv1(self.quant(x)))))
            for i in range(1, 5):
                x = getattr(self, f"layer{i}")(x)
            return self.dequant(self.fc(self.flatten(self.avgpool(x))))

    return ResNet18().eval()


def resnet18_fuse_groups() -> list[list[str]]:
    """conv + bn (+ relu) runs of :func:`resnet18` for ``fuse_modules``."""
    groups = [["conv1", "bn1", "relu"]]
    for i in range(1, 5):
        for b in range(2):
            p = f"layer{i}.{b}"
            groups += [[f"{p}.conv1", f"{p}.bn1", f"{p}.relu"], [f"{p}.conv2", f"{p}.bn2"]]
            if i > 1 and b == 0:
                groups.append([f"{p}.downsample.0", f"{p}.downsample.1"])
    return groups


# --------------------------------------------------------------------- configuration 4


def decoder(rng: np.random.Generator):
    """The decoder's Linears (N(0, 0.02) weights and biases) as a module tree, and the float
    embeddings {"tok": [VOCAB, D], "pos": [PREFILL + DECODE, D]} (host arrays)."""
    import lucid_amd.nn as nn

    def lin(k, n):
        m = nn.Linear(k, n)
        m.weight = nn.Parameter(_host(rng.normal(0, 0.02, (n, k))))
        m.bias = nn.Parameter(_host(rng.normal(0, 0.02, n)))
        return m

    class Layer(nn.Module):
        def __init__(self):
            super().__init__()
            self.qkv = lin(D_MODEL, 3 * D_MODEL)
            self.out = lin(D_MODEL, D_MODEL)
            self.up = lin(D_MODEL, FFN)
            self.down = lin(FFN, D_MODEL)

    class Decoder(nn.Module):
        def __init__(self):
            super().__init__()
            self.layers = nn.Sequential(*[Layer() for _ in range(LAYERS)])
            self.head = lin(D_MODEL, VOCAB)

    glue = {"tok": rng.normal(0, 0.02, (VOCAB, D_MODEL)).astype(np.float32),
            "pos": rng.normal(0, 0.02, (PREFILL + DECODE, D_MODEL)).astype(np.float32)}
    return Decoder().to("gpu"), glue


class DynLinear:
    """One ``nnqd.Linear`` run through the C ABI into caller buffers, allocating nothing per
    call: ``lq_dynamic_quantize_f32`` (live range, per-tensor affine qparams on the module's
    activation grid, codes as c - 128; one launch at decode sizes) -> ``lq_gemm_w8a8`` /
    ``lq_gemm_w8a8_packed`` (M <= 128) with ``LQ_EPI_A_U8S8``, the module's weight codes,
    per-channel scales, cached code sums and bias, float32 out -- the launches of
    ``nnqd.Linear.forward``."""

    def __init__(self, mod, max_rows: int) -> None:
        w = mod._operands()
        self.N, self.K = w.N, w.K
        if w.zero_point is not None:
            raise ValueError("DynLinear: symmetric (zero-point-free) weights expected")
        self.w = w
        self.packed = w.packed()
        self.bias = mod.bias
        qd = mod.act_qdtype
        self.qmin, self.qmax, self.signed = qd.quant_min, qd.quant_max, int(qd.signed)
        if not (0 <= self.qmin and self.qmax <= 255):
            raise ValueError("DynLinear: an unsigned 8-bit activation grid expected")
        self.qp = empty((4,), np.float32, "gpu")  # min, max, scale, zero point
        self.codes = empty((max_rows * self.K,), np.int8, "gpu")
        lib = _C.lib()
        self.mm_bytes = max(lib.lq_dynamic_quantize_workspace_size(max_rows * self.K), 16)
        self.mm_ws = empty((self.mm_bytes,), np.uint8, "gpu")
        self.g_bytes = max(max(lib.lq_gemm_w8a8_workspace_size(m, self.N, self.K) for m in (1, max_rows)), 16)
        self.g_ws = empty((self.g_bytes,), np.uint8, "gpu")
        self.ln_bytes = max(lib.lq_layer_norm_dynamic_quantize_workspace_size(max_rows, self.K), 16)
        self.ln_ws = empty((self.ln_bytes,), np.uint8, "gpu")
        self.gq_bytes = max(lib.lq_gemm_w8a8_dynamic_quantize_workspace_size(max_rows, self.N, self.K), 16)
        self.gq_ws = empty((self.gq_bytes,), np.uint8, "gpu")

    def tensors(self) -> list:
        """Every device tensor a call reads or writes."""
        w = self.w
        return [t for t in (self.qp, self.codes, self.mm_ws, self.g_ws, self.ln_ws, self.gq_ws, self.packed, self.bias,
                            w.codes, w.scale, w.sums) if t is not None]

    EPS = float(np.float32(1e-8))
    LN_FUSED_MAX = 12288  # one-workgroup limit of the fused layer norm + input step

    def __call__(self, x: int, rows: int, y: int, stream) -> None:
        n = rows * self.K
        _C.call("lq_dynamic_quantize_f32", x, n, _C.U8S8, self.qmin, self.qmax, self.EPS, self.qp.data_ptr(),
                self.codes.data_ptr(), self.mm_ws.data_ptr(), self.mm_bytes, stream)
        self.gemm(rows, y, stream)

    def quantize_ln(self, x: int, ldx: int, res, ldres: int, rows: int, stream) -> bool:
        """The input step fused with the LayerNorm before it (x += res first when res is given):
        lq_layer_norm_quantize_f32, the bits of the norm then the input step.  False (nothing
        launched) when the rows exceed one workgroup's limit."""
        if rows * self.K > self.LN_FUSED_MAX:
            return False
        _C.call("lq_layer_norm_quantize_f32", x, ldx, res, ldres, rows, self.K, None, None, np.float32(1e-5),
                _C.U8S8, self.qmin, self.qmax, self.EPS, self.qp.data_ptr(), self.codes.data_ptr(), stream)
        return True

    def quantize_ln_rows(self, x: int, ldx: int, res, ldres: int, rows: int, y: int, stream) -> None:
        """The same step at any row count, the normalized rows stored to ``y`` [rows, K]:
        lq_layer_norm_dynamic_quantize_f32, the bits of lq_(add_)layer_norm_f32 then
        lq_dynamic_quantize_f32 (two launches at prefill sizes)."""
        _C.call("lq_layer_norm_dynamic_quantize_f32", x, ldx, res, ldres, rows, self.K, None, None, np.float32(1e-5),
                y, _C.U8S8, self.qmin, self.qmax, self.EPS, self.qp.data_ptr(), self.codes.data_ptr(),
                self.ln_ws.data_ptr(), self.ln_bytes, stream)

    ONE_LAUNCH_MK, ONE_LAUNCH_MK_LN = 16384, 8192  # lq_dynamic_linear_packed_f32's limits

    def one_launch(self, x: int, ldx: int, res, ldres: int, sum_, src: int, rows: int, y: int, stream,
                   gelu: bool = False) -> bool:
        """The whole forward in one launch (lq_dynamic_linear_packed_f32), the layer norm
        before it folded in for ``src`` DL_LN / DL_ADD_LN (x + res stored to ``sum_``): the
        bits of the norm, the input step and the product.  False (nothing launched) outside its
        sizes (rows <= 16, K % 16 == 0, rows K <= 16384; with a norm K <= 2048, rows K <= 8192)."""
        mk = self.ONE_LAUNCH_MK if src == _C.DL_PLAIN else self.ONE_LAUNCH_MK_LN
        if (self.packed is None or rows > 16 or self.K % 16 or rows * self.K > mk
                or (src != _C.DL_PLAIN and self.K > 2048)):
            return False
        _C.call("lq_dynamic_linear_packed_f32", x, ldx, res, ldres, sum_, self.K, src, None, None, np.float32(1e-5),
                rows, self.K, self.qmin, self.qmax, self.EPS, self.qp.data_ptr(), self.packed.data_ptr(),
                self.w.scale.data_ptr(), self.w.sums.data_ptr(),
                self.bias.data_ptr() if self.bias is not None else None, self.N, y, self.N,
                _C.EPI_GELU if gelu else 0, stream)
        return True

    def gemm_quantize(self, rows: int, y: int, nxt: "DynLinear", stream, gelu: bool = False) -> None:
        """The product into float32 ``y`` [rows, N] and, from it, ``nxt``'s input step (its codes
        and qparams): lq_gemm_w8a8_dynamic_quantize, the bits of :meth:`gemm` followed by
        ``lq_dynamic_quantize_f32`` on ``y``."""
        q = self.qp.data_ptr()
        _C.call("lq_gemm_w8a8_dynamic_quantize", self.codes.data_ptr(), self.K, self.w.codes.data_ptr(), self.K, y,
                rows, self.N, self.K, q + 8, 0, self.w.scale.data_ptr(), 1, q + 12, None, self.w.sums.data_ptr(),
                self.bias.data_ptr() if self.bias is not None else None,
                _C.EPI_A_U8S8 | (_C.EPI_GELU if gelu else 0), _C.U8S8, nxt.qmin, nxt.qmax, nxt.EPS,
                nxt.qp.data_ptr(), nxt.codes.data_ptr(), self.gq_ws.data_ptr(), self.gq_bytes, stream)

    def gemm(self, rows: int, y: int, stream, gelu: bool = False, out_kind: int | None = None) -> None:
        """The int8 product of the codes the last input step left, float32 out (with the tanh
        GELU of the following float module in its epilogue when ``gelu``; ``out_kind``
        ``_C.OUT_F16`` rounds the same float32 values to fp16 for a consumer that would)."""
        q = self.qp.data_ptr()
        sx, zx = q + 8, q + 12
        flags = _C.EPI_A_U8S8 | (_C.EPI_GELU if gelu else 0)
        common = (sx, 0, self.w.scale.data_ptr(), 1, zx, None, self.w.sums.data_ptr(),
                  self.bias.data_ptr() if self.bias is not None else None, None, None, 0, 0,
                  _C.OUT_F32 if out_kind is None else out_kind, flags, self.g_ws.data_ptr(), self.g_bytes, stream)
        if rows <= 128 and self.packed is not None:
            _C.call("lq_gemm_w8a8_packed", self.codes.data_ptr(), self.K, self.packed.data_ptr(), y, self.N, rows,
                    self.N, self.K, *common)
        else:
            _C.call("lq_gemm_w8a8", self.codes.data_ptr(), self.K, self.w.codes.data_ptr(), self.K, y, self.N, rows,
                    self.N, self.K, *common)


class Int8Decoder:
    """Configuration 4 on the device: ``qdec`` (the output of ``quantize_dynamic`` on
    :func:`decoder`) plus its float embeddings, run through the C ABI on preallocated
    buffers.  ``prefill(tokens, stream)`` feeds a [batch, T] prompt from position 0;
    ``decode(stream)`` feeds the previous step's argmax token at the next position.  Both
    leave the last position's logits in ``self.logits`` and its argmax in ``self.next``;
    every launch goes to ``stream``, so either step can be captured into a HIP graph and
    replayed (the position is the device counter ``self.pos``)."""

    def __init__(self, qdec, glue: dict, batch: int = BATCH, max_prompt: int = PREFILL,
                 max_positions: int = PREFILL + DECODE, one_launch: bool = True) -> None:
        self.B, self.Tp, self.Tmax = batch, max_prompt, max_positions
        self.one_launch = one_launch  # decode Linears as lq_dynamic_linear_packed_f32 where it applies
        self.D, self.H, self.hd = D_MODEL, HEADS, D_MODEL // HEADS
        rows = batch * max_prompt
        self.layers = [tuple(DynLinear(getattr(layer, n), rows) for n in ("qkv", "out", "up", "down"))
                       for layer in qdec.layers]
        self.head = DynLinear(qdec.head, batch)
        self.V = self.head.N
        dev = lambda a: tensor(np.ascontiguousarray(a), device="gpu")  # noqa: E731
        self.tok = dev(glue["tok"])
        self.posemb = dev(glue["pos"])
        self.npos = glue["pos"].shape[0]
        f32 = lambda *s: empty(s, np.float32, "gpu")  # noqa: E731
        self.h, self.hn, self.att, self.proj = f32(rows, self.D), f32(rows, self.D), f32(rows, self.D), f32(rows, self.D)
        self.h2 = f32(batch, self.D)  # the residual stream's second buffer for one-launch decode steps
        self.qkv, self.up, self.hl = f32(rows, 3 * self.D), f32(rows, FFN), f32(batch, self.D)
        self.logits = f32(batch, self.V)
        self.q16 = empty((batch, self.H, max_prompt, self.hd), np.float16, "gpu")
        self.att_bytes = max(_C.lib().lq_attention_dynamic_quantize_workspace_size(batch, self.H, max_prompt, self.hd),
                             16)
        self.att_ws = empty((self.att_bytes,), np.uint8, "gpu")  # attention's extrema pairs
        self.cache = [(empty((batch, self.H, self.Tmax, self.hd), np.float16, "gpu"),
                       empty((batch, self.H, self.Tmax, self.hd), np.float16, "gpu")) for _ in self.layers]
        self.prompt = empty((rows,), np.int32, "gpu")
        self.next = empty((batch,), np.int32, "gpu")
        self.pos = empty((1,), np.int32, "gpu")
        self.scale = float(np.float32(1.0 / np.sqrt(self.hd)))
        self._streams: set = set()

    def _use_stream(self, stream) -> None:
        """Tie every buffer and weight the steps touch to ``stream`` (once per stream): when
        this runtime is dropped while work queued there is still running, the allocator does
        not hand the memory out before that work completes (``Tensor.record_stream``)."""
        key = getattr(stream, "value", stream)
        if key is None or key in self._streams:
            return
        self._streams.add(key)
        bufs = [self.tok, self.posemb, self.h, self.h2, self.hn, self.att, self.proj, self.qkv, self.up, self.hl,
                self.logits, self.q16, self.att_ws, self.prompt, self.next, self.pos]
        bufs += [t for kv in self.cache for t in kv]
        bufs += [t for lins in self.layers for lin in lins for t in lin.tensors()] + self.head.tensors()
        for t in bufs:
            t.record_stream(stream)

    def _decode_one_launch(self, stream) -> bool:
        """A decode step whose Linears each run as one launch with the norm before them
        (lq_dynamic_linear_packed_f32): the residual stream alternates between two buffers,
        since the sum is stored while other workgroups still read the old one.  False when the
        sizes fall outside that entry (nothing launched)."""
        B, D, H, hd = self.B, self.D, self.H, self.hd
        normed = [lin for (qkv, _, up, _) in self.layers for lin in (qkv, up)] + [self.head]
        plain = [lin for (_, out, _, down) in self.layers for lin in (out, down)]
        if B > 16 or any(lin.packed is None or lin.K % 16 for lin in normed + plain):
            return False
        if any(B * lin.K > lin.ONE_LAUNCH_MK_LN or lin.K > 2048 for lin in normed):
            return False
        if any(B * lin.K > lin.ONE_LAUNCH_MK for lin in plain):
            return False
        p = self.pos.data_ptr()
        cur, nxt = self.h.data_ptr(), self.h2.data_ptr()
        _C.call("lq_embedding_sum_f32", self.tok.data_ptr(), self.V, self.posemb.data_ptr(), self.npos, D,
                self.next.data_ptr(), B, 1, 0, p, cur, stream)
        proj = self.proj.data_ptr()
        for li, ((qkv, out, up, down), (kc, vc)) in enumerate(zip(self.layers, self.cache)):
            if li == 0:
                qkv.one_launch(cur, D, None, D, None, _C.DL_LN, B, self.qkv.data_ptr(), stream)
            else:
                qkv.one_launch(cur, D, proj, D, nxt, _C.DL_ADD_LN, B, self.qkv.data_ptr(), stream)
                cur, nxt = nxt, cur
            _C.call("lq_kv_append_attention_f16", self.qkv.data_ptr(), B, H, hd, 0, p, self.Tmax, kc.data_ptr(),
                    vc.data_ptr(), np.float32(self.scale), self.att.data_ptr(), stream)
            out.one_launch(self.att.data_ptr(), D, None, D, None, _C.DL_PLAIN, B, proj, stream)
            up.one_launch(cur, D, proj, D, nxt, _C.DL_ADD_LN, B, self.up.data_ptr(), stream, gelu=True)
            cur, nxt = nxt, cur
            down.one_launch(self.up.data_ptr(), FFN, None, FFN, None, _C.DL_PLAIN, B, proj, stream)
        self.head.one_launch(cur, D, proj, D, None, _C.DL_ADD_LN, B, self.logits.data_ptr(), stream)
        _C.call("lq_argmax_next_f32", self.logits.data_ptr(), B, self.V, self.next.data_ptr(), p, 1, stream)
        return True

    def _step(self, tokens: int, n: int, stream) -> None:
        self._use_stream(stream)
        if self.one_launch and n == 1 and tokens == self.next.data_ptr() and self._decode_one_launch(stream):
            return
        B, D, H, hd = self.B, self.D, self.H, self.hd
        M = B * n
        p = self.pos.data_ptr()
        h, hn = self.h.data_ptr(), self.hn.data_ptr()
        _C.call("lq_embedding_sum_f32", self.tok.data_ptr(), self.V, self.posemb.data_ptr(), self.npos, D, tokens,
                M, n, 0, p, h, stream)
        proj, eps = self.proj.data_ptr(), np.float32(1e-5)
        for li, ((qkv, out, up, down), (kc, vc)) in enumerate(zip(self.layers, self.cache)):
            # each residual add that a norm follows runs inside that norm's launch, and at decode
            # sizes the norm runs inside the next Linear's input step (same bits either way)
            res = None if li == 0 else proj
            if not qkv.quantize_ln(h, D, res, D, M, stream):
                qkv.quantize_ln_rows(h, D, res, D, M, hn, stream)
            if n == 1:  # the step's k / v appended and attended in one launch
                qkv.gemm(M, self.qkv.data_ptr(), stream)
                _C.call("lq_kv_append_attention_f16", self.qkv.data_ptr(), B, H, hd, 0, p, self.Tmax, kc.data_ptr(),
                        vc.data_ptr(), np.float32(self.scale), self.att.data_ptr(), stream)
            else:
                # q / k / v are only read as fp16: the product rounds them in its epilogue (the
                # float32 values' fp16 bits) and the append moves half the bytes
                qkv.gemm(M, self.qkv.data_ptr(), stream, out_kind=_C.OUT_F16)
                _C.call("lq_kv_append_h16", self.qkv.data_ptr(), B, n, H, hd, 0, p, self.Tmax, self.q16.data_ptr(),
                        kc.data_ptr(), vc.data_ptr(), stream)
            if n == 1:
                out(self.att.data_ptr(), M, proj, stream)
            else:
                # the attention and the out-projection's input step (its extrema folded where the
                # attention stores them), then the product
                _C.call("lq_attention_dynamic_quantize_f16", self.q16.data_ptr(), kc.data_ptr(), vc.data_ptr(), B,
                        H, n, hd, 0, p, self.Tmax, np.float32(self.scale), self.att.data_ptr(), _C.U8S8, out.qmin,
                        out.qmax, out.EPS, out.qp.data_ptr(), out.codes.data_ptr(), self.att_ws.data_ptr(),
                        self.att_bytes, stream)
                out.gemm(M, proj, stream)
            if not up.quantize_ln(h, D, proj, D, M, stream):
                up.quantize_ln_rows(h, D, proj, D, M, hn, stream)
            if n == 1:
                up.gemm(M, self.up.data_ptr(), stream, gelu=True)  # the GELU in the product's epilogue
                down(self.up.data_ptr(), M, proj, stream)
            else:
                # the up projection (GELU in its epilogue) folds its output's extrema for the down
                # projection's input step
                up.gemm_quantize(M, self.up.data_ptr(), down, stream, gelu=True)
                down.gemm(M, proj, stream)
        # the last position of each sequence: the residual add and layer norm over rows n * D
        # apart (only those rows of h are read again), then the head
        hl, pl = h + (n - 1) * D * 4, proj + (n - 1) * D * 4
        if self.head.quantize_ln(hl, n * D, pl, n * D, B, stream):
            self.head.gemm(B, self.logits.data_ptr(), stream)
        else:
            _C.call("lq_add_layer_norm_f32", hl, n * D, pl, n * D, self.hl.data_ptr(), D, B, D, None, None, eps,
                    stream)
            self.head(self.hl.data_ptr(), B, self.logits.data_ptr(), stream)
        # the greedy token and the position advance in one launch
        _C.call("lq_argmax_next_f32", self.logits.data_ptr(), B, self.V, self.next.data_ptr(), p, n, stream)

    def set_prompt(self, tokens: np.ndarray) -> None:
        """Upload a [batch, T] int prompt (T <= max_prompt) for :meth:`prefill`."""
        tokens = np.ascontiguousarray(tokens, np.int32)
        if tokens.shape[0] != self.B or tokens.shape[1] > self.Tp:
            raise ValueError(f"prompt of shape {tokens.shape} for batch {self.B}, at most {self.Tp} tokens")
        if tokens.min() < 0 or tokens.max() >= self.V:
            raise ValueError("prompt token ids out of the vocabulary")
        self.T = tokens.shape[1]
        _C.call("lq_memcpy_h2d", self.prompt.data_ptr(), tokens.ctypes.data, tokens.nbytes, None)

    def prefill(self, stream) -> None:
        """The prompt from position 0 (the counter is reset first)."""
        _C.call("lq_fill_u32", self.pos.data_ptr(), 0, 1, stream)
        self._step(self.prompt.data_ptr(), self.T, stream)

    def decode(self, stream) -> None:
        """One greedy step: the previous argmax token at the next position."""
        self._step(self.next.data_ptr(), 1, stream)


class Graph:
    """A captured sequence of launches on a created stream, replayable (``lq_graph_*``)."""

    def __init__(self, fn, stream) -> None:
        self.stream = stream
        _C.call("lq_graph_begin_capture", stream)
        try:
            fn(stream)
        finally:
            exe = ctypes.c_void_p()
            _C.call("lq_graph_end_capture", stream, ctypes.byref(exe))
        self.exe = exe

    def launch(self) -> None:
        _C.call("lq_graph_launch", self.exe, self.stream)

    def __del__(self) -> None:
        if getattr(self, "exe", None) is not None and _C._lib is not None:
            _C._lib.lq_graph_destroy(self.exe)


def static_resnet18(batch: int = 32, calib_batches: int = 16, seed: int = 5):
    """ResNet-18 with BatchNorm folded, MinMax-calibrated on
    ``calib_batches`` random batches, converted to the static int8 layers.  Returns the
    quantized model and one device input batch."""
    import lucid_amd as L
    import lucid_amd.quantization as Q
    from lucid_amd.nn.layers import manual_seed

    manual_seed(seed)
    rng = np.random.default_rng(seed)
    fused = Q.fuse_modules(resnet18(rng), resnet18_fuse_groups()).to("gpu")
    prepared = Q.prepare(fused, Q.get_minmax_qconfig())
    for _ in range(calib_batches):
        prepared(L.tensor(rng.standard_normal((batch, 3, 224, 224)).astype(np.float32), device="gpu"))
    qnet = Q.convert(prepared)
    x = L.tensor(rng.standard_normal((batch, 3, 224, 224)).astype(np.float32), device="gpu")
    return qnet, x


def _decoder_eager(n_decode: int) -> None:
    """Configuration 4 launched eagerly on a created stream (no graph): two prefills of the
    8 x 512 prompt, then ``n_decode`` greedy steps, each timed with host clocks around a
    stream synchronize.  For kernel traces: a profiler then sees plain kernel launches."""
    import ctypes
    import time

    import lucid_amd.backends as backends
    from lucid_amd.quantization import quantize_dynamic

    backends.quantized.engine = "reference"
    rng = np.random.default_rng(44)
    dec, glue = decoder(rng)
    rt = Int8Decoder(quantize_dynamic(dec), glue)
    rt.set_prompt(rng.integers(0, VOCAB, (BATCH, PREFILL)))
    st = ctypes.c_void_p()
    _C.call("lq_stream_create", ctypes.byref(st))
    try:
        pre = []
        for _ in range(2):
            t0 = time.perf_counter()
            rt.prefill(st)
            _C.call("lq_stream_synchronize", st)
            pre.append((time.perf_counter() - t0) * 1e3)
        t0 = time.perf_counter()
        for _ in range(n_decode):
            rt.decode(st)
        _C.call("lq_stream_synchronize", st)
        dt = (time.perf_counter() - t0) * 1e3 / max(n_decode, 1)
        print(f"decoder eager: prefill {min(pre):.3f} ms, decode {dt:.4f} ms/step over {n_decode} "
              f"(host launch time included)")
    finally:
        _C.call("lq_stream_destroy", st)


def _main(argv: list[str]) -> None:
    """``python3 -m lucid_amd.bench_configs resnet18 [forwards]``: time the configuration-5
    forward (module dispatch included) after three warm-up forwards;
    ``python3 -m lucid_amd.bench_configs decoder [steps]``: configuration 4 launched eagerly
    (two prefills, then greedy steps); ``resnet18_nhwc``: configuration 5 through
    :class:`Int8ResNet`.  A profiler run wraps any of them."""
    import time

    import lucid_amd as L
    import lucid_amd.backends as backends

    if argv and argv[0] == "decoder":
        _decoder_eager(int(argv[1]) if len(argv) > 1 else 16)
        return
    if not argv or argv[0] not in ("resnet18", "resnet18_nhwc"):
        raise SystemExit("usage: python3 -m lucid_amd.bench_configs resnet18|resnet18_nhwc|decoder [count]")
    n = int(argv[1]) if len(argv) > 1 else 10
    backends.quantized.engine = "reference"  # the per-channel int8 layers
    qnet, x = static_resnet18(calib_batches=4)
    if argv[0] == "resnet18_nhwc":
        qnet = Int8ResNet(qnet, 32)
    for _ in range(3):
        qnet(x)
    L.synchronize()
    ts = []
    for _ in range(n):
        t0 = time.perf_counter()
        qnet(x)
        L.synchronize()
        ts.append((time.perf_counter() - t0) * 1e3)
    ts.sort()
    print(f"resnet18 batch 32: forward median {ts[len(ts) // 2]:.3f} ms over {n}")



class Int8ResNet:
    """Configuration 5's converted network (:func:`static_resnet18`'s output) with its
    activations kept, between the block convolutions, in the padded NHWC layout the int8
    implicit GEMM reads: the stem (QuantStub, then the 7 x 7 convolution) as its modules run
    it, the max pool into that layout (``lq_maxpool2d_i8_to_nhwc``), every block convolution
    through ``lq_conv2d_i8_nhwc`` -- each writing the next one's input with its zero-point
    border, the block's residual ``add_relu`` fused into its second convolution -- the global
    average pool from the layout (``lq_avgpool2d_global_nhwc``), and the fc and DeQuantStub as
    their modules run them.  The per-layer repacking of the input (NCHW to padded NHWC) and the
    separate merge launches of the module forward are gone; the codes, and the result, are the
    module forward's bits.  Buffers are allocated for one batch size; :meth:`forward` can be
    recorded and replayed as one graph (``lucid_amd.graphs.CapturedForward``)."""

    def __init__(self, qnet, batch: int, image: int = 224) -> None:
        from lucid_amd.nn.quantized.linear import out_kind_for

        self.qnet, self.N = qnet, batch
        self.blocks = []
        # the stem's output grid and geometry (7 x 7 / 2, then the 3 x 3 / 2 max pool)
        stem = qnet.conv1
        H = (image + 2 * 3 - 7) // 2 + 1
        self.stem_hw, self.pool_hw = H, (H + 2 - 3) // 2 + 1
        grid = (stem.scale, stem.zero_point, out_kind_for(stem.out_qdtype)[1])
        C, H = stem.out_channels, self.pool_hw
        self.stem_out = empty((batch, self.stem_hw, self.stem_hw, C), np.int8, "gpu")  # NHWC, no border
        self.stem_ws_bytes = max(_C.lib().lq_conv2d_i8_workspace_size(batch, stem.in_channels, image, image, C, 7, 7,
                                                                       2, 2, 3, 3, 3, 3, 1, 1, 1), 16)
        self.stem_ws = empty((self.stem_ws_bytes,), np.uint8, "gpu")
        self.pool_out = self._buffer(C, H)
        cur = self.pool_out
        for li in range(1, 5):
            for blk in getattr(qnet, f"layer{li}"):
                conv1, conv2 = blk.conv1, blk.conv2
                st = conv1.stride[0]
                Ho = (H + 2 - 3) // st + 1
                mid = self._buffer(conv1.out_channels, Ho)
                out = self._buffer(conv2.out_channels, Ho)
                ds = None
                if blk.downsample is not None:
                    ds = (blk.downsample[0], self._buffer(blk.downsample[0].out_channels, Ho))
                self.blocks.append(dict(conv1=conv1, conv2=conv2, skip=blk.skip, ds=ds, x=cur, mid=mid, out=out,
                                        C=C, H=H, Ho=Ho, grid=grid))
                grid = (blk.skip.scale, blk.skip.zero_point, _merge_code(blk.skip.qdtype))
                cur, C, H = out, conv2.out_channels, Ho
        self.final, self.final_c, self.final_hw, self.final_grid = cur, C, H, grid
        self.pooled = empty((batch, C), np.float32, "gpu")
        lib = _C.lib()
        ws = 16
        for b in self.blocks:
            for conv, Cin, Hin in ((b["conv1"], b["C"], b["H"]), (b["conv2"], b["conv1"].out_channels, b["Ho"])):
                k = conv.kernel_size[0]
                ws = max(ws, lib.lq_conv2d_i8_nhwc_workspace_size(batch, Cin, Hin, Hin, conv.out_channels, k, k,
                                                                  conv.stride[0], conv._pads()[0]))
        self.ws_bytes = ws
        self.ws = empty((ws,), np.uint8, "gpu")

    def _buffer(self, C: int, H: int):
        """A padded NHWC activation buffer (border 1) for this batch."""
        return empty((self.N, H + 2, H + 2, C), np.int8, "gpu")

    def _conv(self, conv, x, x_grid, Cin, Hin, y, skip=None, skip_grid=None, merge=None) -> None:
        from lucid_amd.nn.quantized.linear import out_kind_for
        from lucid_amd.quantization._device import on_device

        ops = conv._operands()
        s_in, z_in, code_in = x_grid
        out_kind, _ = out_kind_for(conv.out_qdtype)
        k = conv.kernel_size[0]
        qd = conv.out_qdtype
        b = on_device(conv.bias) if conv.bias is not None else None
        if merge is not None:
            ss, zs, st = skip_grid
            ms, mz, mt = merge.scale, merge.zero_point, _merge_code(merge.qdtype)
            mq = (merge.qdtype.quant_min, merge.qdtype.quant_max)
            mflags = _C.EPI_RELU
        _C.call("lq_conv2d_i8_nhwc", x.data_ptr(), code_in, self.N, Cin, Hin, Hin, 1, Cin, ops.packed.data_ptr(),
                ops.sums.data_ptr(), conv.out_channels, k, k, conv.stride[0], conv._pads()[0], on_device(s_in).data_ptr(),
                on_device(z_in).data_ptr(), ops.scale.data_ptr(), b.data_ptr() if b is not None else None,
                on_device(conv.scale).data_ptr(), on_device(conv.zero_point).data_ptr(), qd.quant_min, qd.quant_max,
                out_kind, _C.EPI_RELU if conv._relu else 0, y.data_ptr(), 1, conv.out_channels,
                skip.data_ptr() if skip is not None else None, st if merge is not None else _C.U8S8,
                on_device(ss).data_ptr() if merge is not None else None,
                on_device(zs).data_ptr() if merge is not None else None,
                on_device(ms).data_ptr() if merge is not None else None,
                on_device(mz).data_ptr() if merge is not None else None,
                mq[0] if merge is not None else 0, mq[1] if merge is not None else 255,
                mt if merge is not None else _C.U8S8, mflags if merge is not None else 0, self.ws.data_ptr(),
                self.ws_bytes, None)

    def forward(self, x):
        from lucid_amd.nn.quantized.linear import out_kind_for
        from lucid_amd.quantization._device import on_device

        qnet = self.qnet
        q = qnet.quant(x).quant_source
        stem = qnet.conv1
        ops = stem._operands()
        C, H = stem.out_channels, self.stem_hw
        out_kind, code = out_kind_for(stem.out_qdtype)
        qd = stem.out_qdtype
        b = on_device(stem.bias) if stem.bias is not None else None
        pt, pb, pl, pr = stem._pads()
        # the stem convolution as its module runs it, its codes written NHWC
        _C.call("lq_conv2d_i8", q.codes.data_ptr(), q.code_type, self.N, stem.in_channels, x.shape[2], x.shape[3],
                ops.packed.data_ptr(), ops.sums.data_ptr(), C, stem.kernel_size[0], stem.kernel_size[1],
                stem.stride[0], stem.stride[1], pt, pb, pl, pr, 1, 1, 1, 0,
                q.scale.data_ptr(), q.zero_point.data_ptr(), ops.scale.data_ptr(),
                b.data_ptr() if b is not None else None, on_device(stem.scale).data_ptr(),
                on_device(stem.zero_point).data_ptr(), qd.quant_min, qd.quant_max, out_kind,
                (_C.EPI_RELU if stem._relu else 0) | _C.CONV_OUT_NHWC, self.stem_out.data_ptr(),
                self.stem_ws.data_ptr(), self.stem_ws_bytes, None)
        _C.call("lq_maxpool2d_i8_nhwc", self.stem_out.data_ptr(), code, on_device(stem.zero_point).data_ptr(),
                self.N, C, H, H, 0, C, self.pool_hw, self.pool_hw, 3, 3, 2, 2, 1, 1, self.pool_out.data_ptr(), 1, C,
                None)
        for b in self.blocks:
            self._conv(b["conv1"], b["x"], b["grid"], b["C"], b["H"], b["mid"])
            c1 = b["conv1"]
            g1 = (c1.scale, c1.zero_point, out_kind_for(c1.out_qdtype)[1])
            if b["ds"] is not None:
                dconv, dbuf = b["ds"]
                self._conv(dconv, b["x"], b["grid"], b["C"], b["H"], dbuf)
                skip, skip_grid = dbuf, (dconv.scale, dconv.zero_point, out_kind_for(dconv.out_qdtype)[1])
            else:
                skip, skip_grid = b["x"], b["grid"]
            self._conv(b["conv2"], b["mid"], g1, c1.out_channels, b["Ho"], b["out"], skip, skip_grid, b["skip"])
        s_f, z_f, t_f = self.final_grid
        _C.call("lq_avgpool2d_global_nhwc", self.final.data_ptr(), t_f, on_device(s_f).data_ptr(),
                on_device(z_f).data_ptr(), self.N, self.final_c, self.final_hw, self.final_hw, 1, self.final_c,
                self.pooled.data_ptr(), None)
        return qnet.dequant(qnet.fc(qnet.flatten(self.pooled.reshape(self.N, self.final_c, 1, 1))))

    __call__ = forward


def _merge_code(qdtype) -> int:
    """Code type a QFunctional of ``qdtype`` stores (the merge's _grid_codes choice)."""
    if qdtype.quant_min >= -128 and qdtype.quant_max <= 127:
        return _C.I8
    return _C.U8S8


if __name__ == "__main__":
    import sys

    _main(sys.argv[1:])
