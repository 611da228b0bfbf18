"""Fused patterns for spiking transformers (Spikformer, config C4).

Reference: models/spikformer_github.py (SPS 175-245, SSA 94-160, MLP 59-92,
Block 163-173).  The reference's substitution leaves Linear -> BatchNorm1d ->
LIF unfused (catfuse/substitute.py:559-567) and runs the attention products
in torch; here every Linear -> BN1d -> LIF is one matrix-core launch with BN
folded into the epilogue affine and the LIF (and a residual add) in the
epilogue, Q, K and V share one launch (their weights concatenated), and the
attention core is one launch per layer (cf_spike_attention_lif).

Token tensors [T, B, N, C] stay token-major: a fused layer keeps its output
only as the fp16 copy [T*B*N, cp] (the next fused layer reads it as an NHWC
image of the N tokens) and returns a lazy fp32 tensor that fills itself on
first outside use.  Membrane states live in the kernels' layouts:
Linear layers [B, C, N], the attention LIF [B, N, C].
"""
from __future__ import annotations

from typing import Optional

import torch
import torch.nn as nn

from catfuse_amd.patterns import (CTFPattern, PartialFusionConvBNLIF, conv_unsupported_reason,
                                  fold_bn, is_lif_node, lif_params)
from catfuse_amd.runtime import (ConvLIFRunner, attach_desc, count_block, count_of, desc_of,
                                 keep_of, lazy_tokens, lif_multistep,
                                 maxpool_nhwc,
                                 pad32, shadow_of, spike_attention_lif, token_membrane,
                                 attention_covers,
                                 token_shadow, token_view)
from catfuse_amd.state import StateBuffer


class FusedLinearBNLIF(CTFPattern):
    """Linear (+bias) -> BatchNorm1d (eval, over the feature dim) -> LIF on
    token tensors x [T, B, N, I] (or [T, B, I]) -> spikes [T, B, N, O]
    (models/spikformer_github.py:126-137).  forward(x, identity) adds a
    residual [T, B, N, O] to the spikes in the same epilogue (the
    `x + f(x)` of a Spikformer block)."""

    def __init__(self, in_features, out_features, bias=True, has_bn=True, bn_eps=1e-5,
                 tau=2.0, v_threshold=1.0, v_reset=0.0, decay_input=True):
        super().__init__()
        self.in_features, self.out_features = int(in_features), int(out_features)
        self.tau, self.v_threshold = float(tau), float(v_threshold)
        self.v_reset = None if v_reset is None else float(v_reset)
        self.decay_input = bool(decay_input)
        self.bn_eps = float(bn_eps)
        self.weight = nn.Parameter(torch.empty(out_features, in_features))
        nn.init.kaiming_normal_(self.weight)
        self.bias = nn.Parameter(torch.zeros(out_features)) if bias else None
        if has_bn:
            self.bn_weight = nn.Parameter(torch.ones(out_features))
            self.bn_bias = nn.Parameter(torch.zeros(out_features))
            self.register_buffer("running_mean", torch.zeros(out_features))
            self.register_buffer("running_var", torch.ones(out_features))
        else:
            self.bn_weight = self.bn_bias = None
            self.register_buffer("running_mean", None)
            self.register_buffer("running_var", None)
        self.state = StateBuffer()
        self._register_state(self.state)
        self._tokens = None   # (B, N) of the last call
        self._runner = None
        self._runner_key = None

    def _param_tensors(self):
        # read from the module's own dicts (attribute lookup of a parameter
        # goes through nn.Module.__getattr__ on every call)
        P, Bf = self._parameters, self._buffers
        return [t for t in (P.get("weight"), P.get("bias"), P.get("bn_weight"), P.get("bn_bias"),
                            Bf.get("running_mean"), Bf.get("running_var")) if t is not None]

    def runner(self) -> ConvLIFRunner:
        key = tuple([(id(t), t._version, t.device) for t in self._param_tensors()])
        if key != self._runner_key:
            with torch.no_grad():
                scale = shift = None
                if self.bn_weight is not None:
                    scale, shift = fold_bn(self.bn_weight, self.bn_bias, self.running_mean,
                                           self.running_var, self.bn_eps)
                w = self.weight.detach().contiguous().view(self.out_features,
                                                           self.in_features, 1, 1)
                self._runner = ConvLIFRunner(w, scale, shift,
                                             None if self.bias is None else self.bias.detach(),
                                             1, 0, self.tau, self.v_threshold, self.v_reset,
                                             self.decay_input)
            self._runner_key = key
        return self._runner

    def forward(self, x, identity=None):
        squeeze = x.ndim == 3
        if squeeze:
            x = x.unsqueeze(2)
            identity = None if identity is None else identity.unsqueeze(2)
        T, B, N, _ = x.shape
        nimg, H, W = token_view(B, N)
        v_in = self.state.peek((nimg, self.out_features, H * W), x.device)
        y, v = self.runner().run_tokens(x, v_in, identity=identity)
        self.state.set(v)
        self.__dict__["_tokens"] = (B, N)   # a plain attribute (no nn.Module hook)
        return y.squeeze(2) if squeeze else y

    def membrane(self):
        """The LIF state after the last call as [B, N, out_features] (None
        after a reset).  Held per launch view image ([nimg, out, H * W],
        runtime.token_view), the layout the kernel reads and writes."""
        v = self.state.tensor
        return None if v is None else token_membrane(v, *self._tokens)

    @classmethod
    def from_sj_modules(cls, linear, bn, lif):
        inst = cls(linear.in_features, linear.out_features, bias=linear.bias is not None,
                   has_bn=bn is not None, bn_eps=bn.eps if bn is not None else 1e-5,
                   **lif_params(lif))
        with torch.no_grad():
            inst.weight.copy_(linear.weight)
            if linear.bias is not None:
                inst.bias.copy_(linear.bias)
            if bn is not None:
                inst.bn_weight.copy_(bn.weight)
                inst.bn_bias.copy_(bn.bias)
                inst.running_mean.copy_(bn.running_mean)
                inst.running_var.copy_(bn.running_var)
        return inst.to(linear.weight.device)

    @classmethod
    def concatenated(cls, triples):
        """One layer computing several Linear -> BN1d -> LIF triples that
        share their input and neuron parameters (Q, K and V): output
        features in the order given."""
        lins = [t[0] for t in triples]
        lps = [lif_params(t[2]) for t in triples]
        if any(lp != lps[0] for lp in lps):
            raise ValueError("concatenated layers need equal LIF parameters")
        eps = {t[1].eps for t in triples}
        if len(eps) != 1 or any(t[1] is None for t in triples):
            raise ValueError("concatenated layers need BatchNorm1d with one eps")
        I = lins[0].in_features
        O = sum(l.out_features for l in lins)
        has_bias = all(l.bias is not None for l in lins)
        inst = cls(I, O, bias=has_bias, has_bn=True, bn_eps=eps.pop(), **lps[0])
        with torch.no_grad():
            inst.weight.copy_(torch.cat([l.weight for l in lins], 0))
            if has_bias:
                inst.bias.copy_(torch.cat([l.bias for l in lins], 0))
            for name, attr in (("bn_weight", "weight"), ("bn_bias", "bias"),
                               ("running_mean", "running_mean"), ("running_var", "running_var")):
                getattr(inst, name).copy_(torch.cat([getattr(t[1], attr) for t in triples], 0))
        return inst.to(lins[0].weight.device)


class CTFSpikformerSSA(CTFPattern):
    """Spiking self-attention: fused QKV Linear-BN1d-LIF (one launch), the
    attention core with attn_lif (one launch), fused proj Linear-BN1d-LIF
    (+ the block's residual).

    The core kernels cover head dims 32 and 64 at any token count below
    65,536 (cf_spike_attention_lif: head dim 32, up to 256 tokens, one
    launch; cf_spike_attention_kv_lif: the others, K^T V then Q (K^T V), e.g.
    spikformer_cifar_tiny's head dim 64 or a 56 x 56 token grid).  Other
    head dims evaluate the same product as two library GEMMs in float64 on
    the GPU (exact: the operands are spikes and every partial sum an
    integer), round once by the scale in fp32 and run the LIF in
    cf_lif_multistep: the same values the kernels produce.  Such calls are
    counted in `gemm_core_calls`."""

    def __init__(self, dim, num_heads, scale, qkv: FusedLinearBNLIF, proj: FusedLinearBNLIF,
                 attn_lif_params: dict):
        super().__init__()
        if dim % num_heads:
            raise ValueError("dim must be a multiple of num_heads")
        self.dim, self.num_heads, self.scale = int(dim), int(num_heads), float(scale)
        self.head_dim = self.dim // self.num_heads
        self.qkv = qkv
        self.proj = proj
        self.attn_lif = dict(attn_lif_params)
        self.attn_state = StateBuffer()
        self._register_state(self.attn_state)
        self._attn_gen = [0]        # calls that published the core's count block
        self._attn_blocks = {}
        self.gemm_core_calls = 0

    def kernel_covers(self, N: int) -> bool:
        return attention_covers(self.head_dim, N)

    def forward(self, x, residual=None):
        T, B, N, C = x.shape
        qkv = self.qkv(x)
        lp = self.attn_lif
        v_in = self.attn_state.peek((B, N, C), x.device)
        nnz = count_of(qkv)
        # With a current count block the kernel takes its zero route on an
        # all-zero copy and reads nothing, so a copy its producer left
        # unwritten (all zero) need not be filled; one that may alias
        # another copy is.
        copy = (token_shadow(qkv, pad32(3 * C), resolve=nnz is None or bool(keep_of(qkv)))
                if self.kernel_covers(N) else None)
        if copy is not None:
            a, v = spike_attention_lif(copy, T, B, N, self.num_heads, (0, C, 2 * C), self.scale,
                                       tau=lp["tau"], v_threshold=lp["v_threshold"],
                                       v_reset=lp["v_reset"], decay_input=lp["decay_input"],
                                       v_in=v_in, nz_out=self._attn_block(x.device),
                                       gen_cell=self._attn_gen, nnz=nnz,
                                       head_dim=self.head_dim)
        else:
            a, v = self._gemm_core(qkv, v_in)
        self.attn_state.set(v)
        return self.proj(a, identity=residual)

    def _gemm_core(self, qkv, v_in):
        """LIF_T(Q (K^T V) * scale) for shapes the core kernel does not cover:
        float64 GEMMs of the spike operands (exact integers), one fp32
        rounding by the scale, cf_lif_multistep over T."""
        T, B, N, C3 = qkv.shape
        C, H, dh = C3 // 3, self.num_heads, self.head_dim
        with torch.no_grad():
            t = qkv.reshape(T, B, N, 3, H, dh).permute(3, 0, 1, 4, 2, 5).double()
            q, k, v = t[0], t[1], t[2]                       # [T, B, H, N, dh]
            kv = torch.matmul(k.transpose(-1, -2).contiguous(), v.contiguous())
            y = torch.matmul(q.contiguous(), kv)             # integers, exact
            z = y.permute(0, 1, 3, 2, 4).reshape(T, B, N, C).float() * self.scale
        lp = self.attn_lif
        self.gemm_core_calls += 1
        return lif_multistep(z.contiguous(), v_in, tau=lp["tau"], v_threshold=lp["v_threshold"],
                             v_reset=lp["v_reset"], decay_input=lp["decay_input"])

    def _attn_block(self, device):
        blk = self._attn_blocks.get(device)
        if blk is None:
            blk = count_block(device)
            self._attn_blocks[device] = blk
        return blk

    @classmethod
    def from_sj_module(cls, ssa):
        qkv = FusedLinearBNLIF.concatenated([(ssa.q, ssa.q_bn, ssa.q_lif),
                                             (ssa.k, ssa.k_bn, ssa.k_lif),
                                             (ssa.v, ssa.v_bn, ssa.v_lif)])
        proj = FusedLinearBNLIF.from_sj_modules(ssa.proj, ssa.proj_bn, ssa.proj_lif)
        return cls(ssa.dim, ssa.num_heads, ssa.scale, qkv, proj, lif_params(ssa.attn_lif))


class CTFSpikformerMLP(CTFPattern):
    def __init__(self, fc1: FusedLinearBNLIF, fc2: FusedLinearBNLIF):
        super().__init__()
        self.fc1, self.fc2 = fc1, fc2

    def forward(self, x, residual=None):
        return self.fc2(self.fc1(x), identity=residual)

    @classmethod
    def from_sj_module(cls, mlp):
        return cls(FusedLinearBNLIF.from_sj_modules(mlp.fc1, mlp.fc1_bn, mlp.fc1_lif),
                   FusedLinearBNLIF.from_sj_modules(mlp.fc2, mlp.fc2_bn, mlp.fc2_lif))


class CTFSpikformerBlock(CTFPattern):
    """x + SSA(x), then x + MLP(x), the adds in proj's and fc2's epilogues
    (models/spikformer_github.py:162-179)."""

    def __init__(self, attn: CTFSpikformerSSA, mlp: CTFSpikformerMLP):
        super().__init__()
        self.attn, self.mlp = attn, mlp

    def forward(self, x):
        x = self.attn(x, residual=x)
        return self.mlp(x, residual=x)

    @classmethod
    def from_sj_block(cls, block):
        return cls(CTFSpikformerSSA.from_sj_module(block.attn),
                   CTFSpikformerMLP.from_sj_module(block.mlp))


class CTFSpikformerSPS(CTFPattern):
    """Spiking patch splitting: fused Conv-BN-LIF stages (MaxPool2d(3, 2, 1)
    after the pooled ones, on the materialised spikes), then the relative
    position Conv-BN-LIF with its input added in the epilogue; the result's
    NHWC copy is the token copy [T*B*N, C] of the output tokens [T, B, N, C]
    (models/spikformer_github.py:181-254)."""

    def __init__(self, stages, pools, rpe):
        super().__init__()
        self.stages = nn.ModuleList(stages)
        self.pools = nn.ModuleList([p if p is not None else nn.Identity() for p in pools])
        self._pooled = [p is not None for p in pools]
        self.rpe = rpe
        self._pool_gen = [[0] for _ in pools]   # calls that published each pool's count
        self._pool_blocks = {}

    def _pool_block(self, i, device):
        blk = self._pool_blocks.get((i, device))
        if blk is None:
            blk = count_block(device)
            self._pool_blocks[(i, device)] = blk
        return blk

    def forward(self, x):
        T, B = x.shape[:2]
        y = x
        for i, (stage, pool, pooled) in enumerate(zip(self.stages, self.pools, self._pooled)):
            if pooled and self._direct_pool(stage, pool, y):
                # analog input: conv, LIF and pool in one launch
                y = self._run_direct_pool(i, stage, y)
                continue
            y = stage(y)
            if pooled:
                k, st, pd = self._pool_geometry(pool)
                yp = None
                if y.is_cuda and 2 * pd <= k and self._plain_pool(pool):
                    # pool the fp16 NHWC copy (exact for spikes), keep it as a copy
                    yp = maxpool_nhwc(y, k, st, pd, self._pool_gen[i],
                                      self._pool_block(i, y.device))
                if yp is None:
                    p = nn.functional.max_pool2d(y.flatten(0, 1), pool.kernel_size,
                                                 pool.stride, pool.padding)
                    yp = p.reshape(T, B, *p.shape[1:])
                y = yp
        r = self.rpe(y, sew_identity=y)
        C, H, W = r.shape[2:]
        copy = shadow_of(r, (T * B, H, W, pad32(C)), resolve=False)
        if copy is None:
            return r.flatten(-2).transpose(-1, -2).contiguous()
        tok = lazy_tokens((T, B, H * W, C), copy, r.device)
        if desc_of(r) is not None:
            # the same copy, as its producer left it
            attach_desc(tok, desc_of(r), keep_of(r))
        if count_of(r) is not None:
            # the same values: the rpe conv's count block describes the tokens
            tok._cf_count = r._cf_count[:3] + (tok._version,)
        return tok

    @staticmethod
    def _pool_geometry(pool):
        st = pool.stride if pool.stride is not None else pool.kernel_size
        return tuple(int(v if isinstance(v, int) else v[0])
                     for v in (pool.kernel_size, st, pool.padding))

    @staticmethod
    def _plain_pool(pool) -> bool:
        """Square window, stride and padding, no dilation, floor mode: the
        geometry the NHWC pool kernels compute; other pools run in torch."""
        def sq(v):
            return isinstance(v, int) or (len(v) == 2 and v[0] == v[1])
        st = pool.stride if pool.stride is not None else pool.kernel_size
        return (sq(pool.kernel_size) and sq(st) and sq(pool.padding)
                and getattr(pool, "dilation", 1) in (1, (1, 1))
                and not getattr(pool, "ceil_mode", False))

    def _direct_pool(self, stage, pool, x) -> bool:
        if not (x.is_cuda and x.dim() == 5 and stage._impl.input_is_analog(x)):
            return False
        if not self._plain_pool(pool):
            return False
        r = stage._impl.runner(stage.spec, stage._ensure_params(), x.device)
        return r.direct_pool_supported(x, self._pool_geometry(pool))

    def _run_direct_pool(self, i, stage, x):
        """The analog first stage in one launch, fp32 on the VALU
        (cf_conv_direct_lif_maxpool).  (cf_conv_stem_lif_maxpool also takes
        this stride-1 3x3 stage on the matrix cores, but measured slower on
        Spikformer-8-384's 224 x 224 x 48 stage: 315 against 278 us per
        step, its LIF over 64 padded channels and recomputed border outputs
        outweighing the cheaper conv.)"""
        stage._impl.check_input(x, stage.spec)
        r = stage._impl.runner(stage.spec, stage._ensure_params(), x.device)
        B = x.shape[1]
        Ho, Wo = r.out_hw(x.shape[3], x.shape[4])
        v_in = stage.state.peek((B, stage.out_channels, Ho, Wo), x.device)
        y, v = r.run_direct_pool(x, v_in, nz_out=self._pool_block(i, x.device),
                                 gen_cell=self._pool_gen[i])
        stage.state.set(v)
        return y

    @classmethod
    def from_sj_module(cls, sps):
        stages, pools = [], []
        for i in range(4):
            conv, bn, lif = (getattr(sps, f"{n}{i}") for n in ("conv", "bn", "lif"))
            stages.append(PartialFusionConvBNLIF.from_sj_modules(conv, bn, lif))
            pools.append(getattr(sps, f"pool{i}", None))
        rpe = PartialFusionConvBNLIF.from_sj_modules(sps.rpe_conv, sps.rpe_bn, sps.rpe_lif)
        return cls(stages, pools, rpe)


def _linear_bn_lif_site(owner, name) -> bool:
    """owner.<name> is an nn.Linear, owner.<name>_bn a BatchNorm1d over its
    outputs and owner.<name>_lif an LIF neuron."""
    lin = getattr(owner, name, None)
    bn = getattr(owner, name + "_bn", None)
    return (isinstance(lin, nn.Linear) and isinstance(bn, nn.BatchNorm1d)
            and bn.num_features == lin.out_features and is_lif_node(getattr(owner, name + "_lif", None)))


def is_spikformer_block(m) -> bool:
    """A Spikformer block (models/spikformer_github.py:162-179) whose every
    neuron is LIF: attn with q/k/v/proj Linear-BN1d-LIF sites, attn_lif,
    num_heads and scale; mlp with fc1/fc2 sites.  Blocks with other neurons
    (IF, PLIF, ...) stay unfused."""
    attn, mlp = getattr(m, "attn", None), getattr(m, "mlp", None)
    if attn is None or mlp is None:
        return False
    if not all(_linear_bn_lif_site(attn, n) for n in ("q", "k", "v", "proj")):
        return False
    if not (is_lif_node(getattr(attn, "attn_lif", None)) and hasattr(attn, "num_heads")
            and hasattr(attn, "scale")):
        return False
    d = attn.q.in_features
    heads = int(attn.num_heads)
    if heads <= 0 or d % heads or any(getattr(attn, n).in_features != d or
                                      getattr(attn, n).out_features != d
                                      for n in ("q", "k", "v", "proj")):
        return False
    # Q, K and V share one launch: equal neuron parameters and BN eps
    lps = [lif_params(getattr(attn, n + "_lif")) for n in ("q", "k", "v")]
    if any(lp != lps[0] for lp in lps) or \
            len({getattr(attn, n + "_bn").eps for n in ("q", "k", "v")}) != 1:
        return False
    return (_linear_bn_lif_site(mlp, "fc1") and _linear_bn_lif_site(mlp, "fc2")
            and mlp.fc1.in_features == d and mlp.fc2.out_features == d)


def is_spikformer_sps(m) -> bool:
    """A spiking patch splitter (models/spikformer_github.py:181-254) with
    conv{0..3} / bn{0..3} / lif{0..3} and rpe_conv / rpe_bn / rpe_lif sites
    the fused kernels compute (LIF neurons, supported convs) and pool{i}
    either absent/None or a MaxPool2d."""
    names = [f"{i}" for i in range(4)]
    for conv, bn, lif in [(f"conv{i}", f"bn{i}", f"lif{i}") for i in names] + \
            [("rpe_conv", "rpe_bn", "rpe_lif")]:
        c = getattr(m, conv, None)
        if not (isinstance(c, nn.Conv2d) and conv_unsupported_reason(c) is None
                and isinstance(getattr(m, bn, None), nn.BatchNorm2d)
                and is_lif_node(getattr(m, lif, None))):
            return False
    return all(getattr(m, f"pool{i}", None) is None or isinstance(getattr(m, f"pool{i}"),
                                                                 nn.MaxPool2d) for i in names)


__all__ = ["FusedLinearBNLIF", "CTFSpikformerSSA", "CTFSpikformerMLP", "CTFSpikformerBlock",
           "CTFSpikformerSPS", "is_spikformer_block", "is_spikformer_sps"]
