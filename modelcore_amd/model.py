"""The model around the KV path: a config tree, the transformer that calls the cached-attention
operator, and the ``ModelManager`` surface that builds it and its caches.

This is the caller side of the path (modelcore/model.py, modelcore/components/*,
modelcore/manager.py:111-119 and :286-299), restated for the architectures the KV path serves:
token embedding (wte -> compute dtype -> RMSNorm), pre-norm residual blocks whose mixer is GQA
attention with RoPE (base 100000), parameterless QK RMSNorm and a x1.2 scale on q and k, optional
sliding windows and cross-layer KV sharing (``kv_slot`` / ``produces_kv``), the ``output_gate``
feature, gated or plain MLPs, and an lm_head with vocab crop and tanh softcap. The module names
follow the reference's v3 state-dict keys (``embedding.wte``, ``body.blocks.<i>.mixer.c_q``,
``body.blocks.<i>.ffn.gate_proj``, ``body.blocks.<i>.mixer.features.output_gate.proj``,
``unembedding.lm_head``), so a reference state dict loads as is.

Attention goes through ``modelcore_amd.kernels.flash_attn.flash_attn``: the HIP kernels, on a ROCm
device only. A different operator namespace with the same two functions can be passed as
``attention=`` (the tests pass the CPU oracle to check this module's own arithmetic on the CPU).

Parameters are created in fp32 and cast to the activation dtype at every matmul, as the reference's
Linear does (modelcore/components/linear.py:13-14); the token embedding is stored in the compute
dtype (modelcore/components/embedding.py:64-71).
"""
from __future__ import annotations

from dataclasses import dataclass, field

import torch
import torch.nn as nn
import torch.nn.functional as F

from modelcore_amd.cache import KVCache, PackedPrefill
from modelcore_amd.runtime import Runtime

TYPE_KEY = "#type"


# -----------------------------------------------------------------------------------------------
# Config tree (the subset of modelcore/config/spec.py this path builds)
# -----------------------------------------------------------------------------------------------
@dataclass
class ComponentSpec:
    type: str
    params: dict = field(default_factory=dict)

    @staticmethod
    def from_dict(d):
        if isinstance(d, ComponentSpec):
            return d
        params = {}
        for key, value in d.items():
            if key == TYPE_KEY or key.startswith("//"):
                continue
            params[key] = _spec_tree(value)
        return ComponentSpec(d[TYPE_KEY], params)


def _spec_tree(value):
    if isinstance(value, dict) and TYPE_KEY in value:
        return ComponentSpec.from_dict(value)
    if isinstance(value, list):
        return [_spec_tree(v) for v in value]
    return value


@dataclass
class ModelConfig:
    sequence_len: int
    vocab_size: int
    n_embd: int
    pad_vocab_size_to: int = 64
    template: str = "base"
    shared: dict = field(default_factory=dict)
    input: ComponentSpec | None = None
    body: ComponentSpec | None = None
    output: ComponentSpec | None = None

    @property
    def padded_vocab_size(self):
        m = self.pad_vocab_size_to
        return ((self.vocab_size + m - 1) // m) * m

    @staticmethod
    def from_dict(d):
        """A v3 config dict (``"#type"`` keys) -> ModelConfig."""
        return ModelConfig(
            sequence_len=d["sequence_len"], vocab_size=d["vocab_size"], n_embd=d["n_embd"],
            pad_vocab_size_to=d.get("pad_vocab_size_to", 64), template=d.get("template", "base"),
            shared={k: ComponentSpec.from_dict(v) for k, v in d.get("shared", {}).items()},
            input=ComponentSpec.from_dict(d["input"]), body=ComponentSpec.from_dict(d["body"]),
            output=ComponentSpec.from_dict(d["output"]))


@dataclass
class AttentionLayerSpec:
    """What a KV cache needs from one attention layer (modelcore/config/spec.py:41-56)."""
    n_head: int
    n_kv_head: int
    head_dim: int
    window: int
    kv_slot: int


# -----------------------------------------------------------------------------------------------
# Components
# -----------------------------------------------------------------------------------------------
def _product(x, w, skinny, partial=False):
    """x . w^T: the decode-sized HIP kernel when asked for and the shapes suit it (with
    ``partial``, its unsummed K-split partials, for a consumer that sums them), else F.linear
    (the reference's call, modelcore/components/linear.py:14)."""
    if skinny:
        from modelcore_amd.kernels import linear as lin
        if lin.supported(x, w):
            return lin.linear_bf16_partials(x, w) if partial else lin.linear_bf16(x, w)
    return F.linear(x, w)


class Linear(nn.Linear):
    """fp32 master weight, cast to the activation dtype at every call -- or, after
    ``Model.cache_inference_weights``, read from a copy cast once (the same values, without the
    per-call cast traffic)."""
    _cast = None
    _in_stack = False  # its cached rows live only in a stacked copy (gate/up interleaved)
    skinny = False  # set by Model.use_skinny_gemm
    partial = False  # set by Model.set_fused_residual: may return the product's partials

    def forward(self, x):
        w = self._cast
        if w is None or w.dtype != x.dtype:
            w = self.weight.to(dtype=x.dtype)
        return _product(x, w, self.skinny, self.partial)


class RMSNorm(nn.Module):
    """Parameterless RMSNorm over the last dim; eps=None is torch's default (the dtype's epsilon)."""

    def __init__(self, eps=None):
        super().__init__()
        self.eps = eps

    def init_weights(self):
        pass

    def forward(self, x):
        return F.rms_norm(x, (x.size(-1),), eps=self.eps)


def rope_tables(n_pos, head_dim, device, dtype, base=100000):
    """cos/sin of the half-split rotation, (1, n_pos, 1, head_dim/2), computed in fp32 then cast
    (modelcore/components/rope.py:15-27)."""
    inv_freq = 1.0 / (base ** (torch.arange(0, head_dim, 2, dtype=torch.float32, device=device)
                                / head_dim))
    angles = torch.outer(torch.arange(n_pos, dtype=torch.float32, device=device), inv_freq)
    return (angles.cos().to(dtype)[None, :, None, :], angles.sin().to(dtype)[None, :, None, :])


def rotate(x, cos, sin):
    """Rotation of (first half, second half) of the last dim by -theta
    (modelcore/components/rope.py:4-12)."""
    half = x.shape[3] // 2
    a, b = x[..., :half], x[..., half:]
    return torch.cat([a * cos + b * sin, a * (-sin) + b * cos], 3)


class Rotary(nn.Module):
    """Owns the cos/sin tables (sequence_len * over_compute positions) and finds each query's
    position from the cache: the shared position when the cache is uniform, a per-row gather of
    cache_seqlens when it is right-ragged (modelcore/components/rotary.py:43-67)."""

    def __init__(self, head_dim, sequence_len, over_compute, runtime):
        super().__init__()
        self.head_dim = head_dim
        self.runtime = runtime
        self.n_pos = sequence_len * over_compute
        cos, sin = rope_tables(self.n_pos, head_dim, torch.empty(0).device, runtime.compute_dtype)
        self.register_buffer("cos", cos, persistent=False)
        self.register_buffer("sin", sin, persistent=False)

    @torch.no_grad()
    def init_weights(self):
        self.cos, self.sin = rope_tables(self.n_pos, self.head_dim, self.cos.device,
                                         self.runtime.compute_dtype)

    def _cos_sin(self, T, kv_cache):
        pos = 0 if kv_cache is None else kv_cache.uniform_pos()
        if pos is not None:
            assert pos + T <= self.cos.size(1), \
                f"Sequence length grew beyond the rotary embeddings cache: {pos + T} > {self.cos.size(1)}"
            return self.cos[:, pos:pos + T], self.sin[:, pos:pos + T]
        idx = kv_cache.cache_seqlens.to(torch.long)[:, None] + torch.arange(
            T, device=kv_cache.cache_seqlens.device)
        # One host read, as in the reference: an index past the table must fail here, not in the
        # gather kernel.
        assert int(idx.max().item()) < self.cos.size(1), \
            f"Sequence length grew beyond the rotary embeddings cache: {int(idx.max().item()) + 1} > {self.cos.size(1)}"
        B = idx.size(0)
        flat = idx.reshape(-1)
        return (self.cos[0].index_select(0, flat).view(B, T, 1, -1),
                self.sin[0].index_select(0, flat).view(B, T, 1, -1))

    def check_positions(self, T, kv_cache):
        """The position asserts of _cos_sin without building the windows, for the fused path
        that reads positions on the device: free when the cache is uniform, one host read when it
        is ragged (as in the reference, modelcore/components/rotary.py:50-62)."""
        pos = kv_cache.uniform_pos()
        if pos is not None:
            assert pos + T <= self.cos.size(1), \
                f"Sequence length grew beyond the rotary embeddings cache: {pos + T} > {self.cos.size(1)}"
            return
        last = int(kv_cache.cache_seqlens.max().item()) + T - 1
        assert last < self.cos.size(1), \
            f"Sequence length grew beyond the rotary embeddings cache: {last + 1} > {self.cos.size(1)}"

    def packed_cos_sin(self, positions):
        """cos/sin at each token's own position, (1, N, 1, head_dim/2), for a packed forward of
        several prompts (PackedPrefill); positions are host-known to fit the table."""
        return (self.cos[0, :, 0].index_select(0, positions)[None, :, None, :],
                self.sin[0, :, 0].index_select(0, positions)[None, :, None, :])

    def forward(self, q, k, kv_cache):
        cos, sin = self._cos_sin(q.size(1), kv_cache)
        return rotate(q, cos, sin), rotate(k, cos, sin)

    def apply_to_q(self, q, kv_cache):
        cos, sin = self._cos_sin(q.size(1), kv_cache)
        return rotate(q, cos, sin)


class OutputGate(nn.Module):
    """y * sigmoid(W . x[..., :in_channels]) per head, per element or per block of outputs, between
    the attention operator and c_proj (modelcore/components/features.py:46-88)."""

    def __init__(self, n_embd, n_head, head_dim, granularity, block_size=None, in_channels=None):
        super().__init__()
        self.in_channels = n_embd if in_channels is None else in_channels
        if granularity == "head":
            self.gates_per_head = 1
        elif granularity == "element":
            self.gates_per_head = head_dim
        elif granularity == "block":
            assert head_dim % block_size == 0, \
                f"head_dim ({head_dim}) must be divisible by block_size ({block_size})"
            self.gates_per_head = head_dim // block_size
        else:
            raise ValueError(f"unknown output_gate granularity {granularity!r}")
        self.proj = Linear(self.in_channels, n_head * self.gates_per_head, bias=False)

    @torch.no_grad()
    def init_weights(self):
        s = 3 ** 0.5 * self.in_channels ** -0.5
        nn.init.uniform_(self.proj.weight, -s, s)

    def forward(self, y, x):
        B, T, H, D = y.shape
        G = self.gates_per_head
        gate = torch.sigmoid(self.proj(x[..., :self.in_channels])).view(B, T, H, G, 1)
        return (y.reshape(B, T, H, G, D // G) * gate).view(B, T, H, D)


class Attention(nn.Module):
    """GQA attention with RoPE, QK-norm and x1.2 on q and k, calling the cached-attention operator
    (modelcore/components/attention.py:53-184). A layer with produces_kv=False has no c_k/c_v and
    reads the producer's already rotated/normed/scaled K/V from the per-forward kv_bus; it still
    passes them to the operator, which rewrites identical values at the same positions."""

    def __init__(self, n_embd, n_head, n_kv_head, head_dim, window, kv_slot, produces_kv,
                 features, rope, norm, attention, epilogue=None):
        super().__init__()
        if head_dim is None:
            assert n_embd % n_head == 0
            head_dim = n_embd // n_head
        assert n_kv_head <= n_head and n_head % n_kv_head == 0
        if not produces_kv and kv_slot is None:
            raise ValueError("produces_kv=False requires an explicit kv_slot")
        self.n_embd, self.n_head, self.n_kv_head, self.head_dim = n_embd, n_head, n_kv_head, head_dim
        self.window = window
        self._kv_slot = kv_slot
        self.kv_slot = kv_slot
        self.produces_kv = produces_kv
        self.rope, self.norm, self.attention = rope, norm, attention
        # RoPE + QK-norm + x1.2 + append in one launch (modelcore_amd.kernels.qk_epilogue) when
        # decoding with a cache; None, or fuse_epilogue = False, runs the reference's separate ops.
        self.epilogue = epilogue
        self.fuse_epilogue = True
        self._qkv = None  # [W_q; W_k; W_v] in the compute dtype, set by cache_inference_weights
        self.c_q = Linear(n_embd, n_head * head_dim, bias=False)
        self.c_k = Linear(n_embd, n_kv_head * head_dim, bias=False) if produces_kv else None
        self.c_v = Linear(n_embd, n_kv_head * head_dim, bias=False) if produces_kv else None
        self.c_proj = Linear(n_head * head_dim, n_embd, bias=False)
        self.features = nn.ModuleDict()
        for spec in features or []:
            if spec.type != "output_gate":
                raise NotImplementedError(f"attention feature {spec.type!r} is not supported")
            self.features["output_gate"] = OutputGate(n_embd, n_head, head_dim, **spec.params)

    def bind_layer(self, layer_idx):
        self.layer_idx = layer_idx
        self.kv_slot = layer_idx if self._kv_slot is None else self._kv_slot

    @torch.no_grad()
    def init_weights(self):
        s = 3 ** 0.5 * self.n_embd ** -0.5
        nn.init.uniform_(self.c_q.weight, -s, s)
        if self.produces_kv:
            nn.init.uniform_(self.c_k.weight, -s, s)
            nn.init.uniform_(self.c_v.weight, -s, s)
        nn.init.zeros_(self.c_proj.weight)
        for f in self.features.values():
            f.init_weights()

    def layer_spec(self):
        return AttentionLayerSpec(self.n_head, self.n_kv_head, self.head_dim, self.window,
                                  self.kv_slot)

    def _project(self, x):
        """q, k, v (k = v = None for a consumer layer) as (B, T, heads, D) views; one product
        against the stacked [W_q; W_k; W_v] when the inference weights are cached (the same dot
        products as three separate ones, read in one pass over the weights)."""
        B, T, _ = x.size()
        Hq, Hk, D = self.n_head * self.head_dim, self.n_kv_head * self.head_dim, self.head_dim
        if self._qkv is not None and self._qkv.dtype == x.dtype:
            qkv = _product(x, self._qkv, self.c_q.skinny)
            q = qkv[..., :Hq].view(B, T, self.n_head, D)
            k = qkv[..., Hq:Hq + Hk].view(B, T, self.n_kv_head, D)
            v = qkv[..., Hq + Hk:].view(B, T, self.n_kv_head, D)
            return q, k, v
        q = self.c_q(x).view(B, T, self.n_head, D)
        if not self.produces_kv:
            return q, None, None
        return (q, self.c_k(x).view(B, T, self.n_kv_head, D),
                self.c_v(x).view(B, T, self.n_kv_head, D))

    qkv_partial = False  # set by Model.set_fused_residual

    def _qkv_partials(self, x):
        """The stacked QKV product as unsummed K-split partials, when the fused pre-attention
        step can sum them itself (the native epilogue, bf16, decode-sized rows), else None."""
        if not (self.qkv_partial and self.produces_kv and self._qkv is not None
                and self._qkv.dtype == x.dtype and self.c_q.skinny
                and self.epilogue is _default_epilogue()):
            return None
        from modelcore_amd.kernels import linear as lin
        return lin.linear_bf16_partials(x, self._qkv) if lin.supported(x, self._qkv) else None

    def fuses_epilogue(self, kv_cache):
        """Whether forward() with this cache takes the fused pre-attention step, whose RoPE reads
        each row's position from cache_seqlens on the device (the separate ops slice the tables
        at the host-side position instead)."""
        return kv_cache is not None and self.epilogue is not None and self.fuse_epilogue \
            and isinstance(self.norm, RMSNorm) and not isinstance(kv_cache, PackedPrefill) \
            and self.head_dim <= 256  # the fused step's kernel covers head dims up to 256

    def forward(self, x, kv_cache, kv_bus):
        B, T, _ = x.size()
        if isinstance(kv_cache, PackedPrefill):
            return self._forward_packed(x, kv_cache, kv_bus)
        fused = self.fuses_epilogue(kv_cache)
        if fused:
            part = self._qkv_partials(x)
            if part is not None:
                return self._forward_fused(x, None, None, None, kv_cache, kv_bus, part)
        q, k, v = self._project(x)
        if fused:
            return self._forward_fused(x, q, k, v, kv_cache, kv_bus)
        if self.produces_kv:
            q, k = self.rope(q, k, kv_cache)
            q, k = self.norm(q), self.norm(k)
            q, k = q * 1.2, k * 1.2
            kv_bus[self.kv_slot] = (k, v)
        else:
            k, v = kv_bus[self.kv_slot]
            q = self.norm(self.rope.apply_to_q(q, kv_cache)) * 1.2
        window_size = (self.window, 0)
        if kv_cache is None:
            y = self.attention.flash_attn_func(q, k, v, causal=True, window_size=window_size)
        else:
            k_cache, v_cache = kv_cache.get_slot_cache(self.kv_slot)
            y = self.attention.flash_attn_with_kvcache(q, k_cache, v_cache, k=k, v=v,
                                                       cache_seqlens=kv_cache.cache_seqlens,
                                                       causal=True, window_size=window_size,
                                                       **self._extensions(kv_cache))
        if "output_gate" in self.features:
            y = self.features["output_gate"](y, x)
        return self.c_proj(y.contiguous().view(B, T, -1))

    def _forward_packed(self, x, packed, kv_bus):
        """The layer over several prompts packed along one sequence (x is (1, total, n_embd)):
        projections on the real tokens only, RoPE at each token's position within its prompt,
        QK-norm and x1.2 as the reference's separate ops, then the varlen operator appends each
        prompt's K/V into its own cache row and attends there."""
        _, T, _ = x.size()
        q, k, v = self._project(x)
        cos, sin = self.rope.packed_cos_sin(packed.positions)
        if self.produces_kv:
            q, k = rotate(q, cos, sin), rotate(k, cos, sin)
            q, k = self.norm(q) * 1.2, self.norm(k) * 1.2
            kv_bus[self.kv_slot] = (k, v)
        else:
            k, v = kv_bus[self.kv_slot]
            q = self.norm(rotate(q, cos, sin)) * 1.2
        k_cache, v_cache = packed.get_slot_cache(self.kv_slot)
        y = self.attention.flash_attn_varlen_with_kvcache(
            q[0], k_cache, v_cache, k=k[0], v=v[0], cache_seqlens=packed.cache_seqlens,
            cu_seqlens=packed.cu_seqlens, max_seqlen=packed.max_seqlen, rows=packed.rows,
            causal=True, window_size=(self.window, 0)).unsqueeze(0)
        if "output_gate" in self.features:
            y = self.features["output_gate"](y, x)
        return self.c_proj(y.contiguous().view(1, T, -1))

    def _extensions(self, kv_cache):
        """Operator keywords beyond the reference's, for an operator that takes them: the
        cache's shared prompt prefix (rows replicated by KVCache.prefill), so the decode reads
        it from row 0 for every row (same values, served by the caches)."""
        shared = getattr(kv_cache, "shared_prefix", 0)
        if shared and "shared_prefix" in getattr(self.attention, "EXTENSIONS", ()):
            return {"shared_prefix": shared}
        return {}

    def _forward_fused(self, x, q, k, v, kv_cache, kv_bus, qkv_part=None):
        """The same layer with the pre-attention ops fused: a producer rotates, norms and scales
        q and k and appends k, v to its slot in one launch; a KV-sharing consumer finds them there
        already (the reference's consumer re-appends identical values, attention.py:70-80), so it
        transforms q only. Then the operator runs without an append."""
        B, T, _ = x.size()
        self.rope.check_positions(T, kv_cache)
        k_cache, v_cache = kv_cache.get_slot_cache(self.kv_slot)
        seqlens = kv_cache.cache_seqlens
        if qkv_part is not None:
            from modelcore_amd.kernels.qk_epilogue import rope_norm_scale_append_partials
            q = rope_norm_scale_append_partials(qkv_part, self.n_head, self.n_kv_head,
                                                self.rope.cos, self.rope.sin, seqlens, k_cache,
                                                v_cache, eps=self.norm.eps, scale=1.2)
            kv_bus[self.kv_slot] = None
        elif self.produces_kv:
            q = self.epilogue(q, self.rope.cos, self.rope.sin, seqlens, k, v, k_cache, v_cache,
                              eps=self.norm.eps, scale=1.2)
            kv_bus[self.kv_slot] = None  # consumers read the slot itself
        else:
            q = self.epilogue(q, self.rope.cos, self.rope.sin, seqlens, eps=self.norm.eps,
                              scale=1.2)
        y = self.attention.flash_attn_with_kvcache(q, k_cache, v_cache, cache_seqlens=seqlens,
                                                   causal=True, window_size=(self.window, 0),
                                                   **self._extensions(kv_cache))
        if "output_gate" in self.features:
            y = self.features["output_gate"](y, x)
        return self.c_proj(y.contiguous().view(B, T, -1))


_ACTIVATIONS = {"silu": F.silu, "gelu": F.gelu, "relu": F.relu,
                "relu2": lambda x: F.relu(x).square()}


class GatedMLP(nn.Module):
    """down(act(gate(x)) * up(x)) (modelcore/components/mlp.py:64-90)."""

    def __init__(self, n_embd, activation, hidden_dim):
        super().__init__()
        self.n_embd = n_embd
        self.activation = activation
        self.act = _ACTIVATIONS[activation]
        self.gate_proj = Linear(n_embd, hidden_dim, bias=False)
        self.up_proj = Linear(n_embd, hidden_dim, bias=False)
        self.down_proj = Linear(hidden_dim, n_embd, bias=False)
        self.hidden_dim = hidden_dim
        self._gate_up = None  # [W_gate; W_up] in the compute dtype, set by cache_inference_weights
        self._gate_up_blocked = False  # rows in 64-row blocks (linear.interleave_gate_up)

    @torch.no_grad()
    def init_weights(self):
        s = 3 ** 0.5 * self.n_embd ** -0.5
        nn.init.uniform_(self.gate_proj.weight, -s, s)
        nn.init.uniform_(self.up_proj.weight, -s, s)
        nn.init.zeros_(self.down_proj.weight)

    def forward(self, x):
        if self._gate_up is not None and self._gate_up.dtype == x.dtype:
            if self._gate_up_blocked:
                from modelcore_amd.kernels import linear as lin
                if self.gate_proj.skinny and self.activation == "silu" \
                        and lin.gated_supported(x, self._gate_up):
                    return self.down_proj(lin.linear_bf16_gated(x, self._gate_up))
                w = self._gate_up if self._gate_up.dim() == 2 else lin.untile_weight(self._gate_up)
                out = _product(x, w, self.gate_proj.skinny)
                gate, up = lin.split_gate_up(out)
                return self.down_proj((self.act(gate) * up).reshape(*out.shape[:-1],
                                                                    self.hidden_dim))
            gate, up = _product(x, self._gate_up, self.gate_proj.skinny).split(self.hidden_dim,
                                                                              dim=-1)
            return self.down_proj(self.act(gate) * up)
        return self.down_proj(self.act(self.gate_proj(x)) * self.up_proj(x))


class MLP(nn.Module):
    """c_proj(act(c_fc(x))) (modelcore/components/mlp.py:37-61)."""

    def __init__(self, n_embd, activation, hidden_dim):
        super().__init__()
        self.n_embd = n_embd
        self.act = _ACTIVATIONS[activation]
        self.c_fc = Linear(n_embd, hidden_dim, bias=False)
        self.c_proj = Linear(hidden_dim, n_embd, bias=False)

    @torch.no_grad()
    def init_weights(self):
        s = 3 ** 0.5 * self.n_embd ** -0.5
        nn.init.uniform_(self.c_fc.weight, -s * 0.4, s * 0.4)
        nn.init.zeros_(self.c_proj.weight)

    def forward(self, x):
        return self.c_proj(self.act(self.c_fc(x)))


class Block(nn.Module):
    """x + mixer(norm(x)), then x + ffn(norm(x)) (modelcore/components/block.py:54-60)."""

    def __init__(self, layer_idx, mixer, ffn, norm):
        super().__init__()
        self.layer_idx = layer_idx
        self.mixer = mixer
        self.mixer.bind_layer(layer_idx)
        self.ffn = ffn
        self.norm = norm

    @torch.no_grad()
    def init_weights(self):
        self.mixer.init_weights()
        self.ffn.init_weights()

    fuse_residual = False  # set by Model.set_fused_residual

    def forward(self, x, kv_cache, kv_bus):
        x = x + self.mixer(self.norm(x), kv_cache, kv_bus)
        return x + self.ffn(self.norm(x))

    def forward_carry(self, x, h, kv_cache, kv_bus):
        """forward(), also returning norm(x) of its output, which the next block's mixer (or the
        lm_head) takes as is; h = norm(x) of the input when the previous block made it. Each
        residual add and the norm after it run as one launch (residual_rmsnorm), which also sums
        the K-split partials of the projection before it."""
        if h is None:
            h = self.norm(x)
        x, h = self._residual(x, self.mixer(h, kv_cache, kv_bus))
        return self._residual(x, self.ffn(h))

    def _residual(self, x, f):
        from modelcore_amd.kernels import residual
        from modelcore_amd.kernels.linear import Partials
        if isinstance(f, Partials) or residual.supported(x) and x.numel() // x.shape[-1] <= 64:
            return residual.residual_rmsnorm(x, f, self.norm.eps)
        x = x + f
        return x, self.norm(x)


class Stack(nn.Module):
    """The layer loop; one fresh kv_bus per forward (modelcore/composers/stack.py:35-42)."""

    def __init__(self, blocks):
        super().__init__()
        self.blocks = nn.ModuleList(blocks)

    @torch.no_grad()
    def init_weights(self):
        for block in self.blocks:
            block.init_weights()

    def forward(self, x, kv_cache):
        return self.forward_carry(x, kv_cache)[0]

    def forward_carry(self, x, kv_cache):
        """The layer loop, also returning norm(x) of the output when the last block made it
        (blocks with fused residual steps), else None."""
        kv_bus = {}
        h = None
        for block in self.blocks:
            if block.fuse_residual:
                x, h = block.forward_carry(x, h, kv_cache, kv_bus)
            else:
                x, h = block(x, kv_cache, kv_bus), None
        return x, h


class TokenEmbedding(nn.Module):
    """wte lookup, cast to the compute dtype, norm (modelcore/components/embedding.py:51-79)."""

    def __init__(self, padded_vocab_size, n_embd, norm, runtime, smear=False):
        super().__init__()
        if smear:
            raise NotImplementedError("token_embedding smear is not supported")
        self.runtime = runtime
        self.norm = norm
        self.wte = nn.Embedding(padded_vocab_size, n_embd)

    @torch.no_grad()
    def init_weights(self):
        nn.init.normal_(self.wte.weight, mean=0.0, std=0.8)
        self.wte.to(dtype=self.runtime.compute_dtype)

    def forward(self, idx):
        return self.norm(self.wte(idx).to(self.runtime.compute_dtype))


class LMHead(nn.Module):
    """norm, projection, vocab crop, fp32, softcap * tanh(x / softcap)
    (modelcore/components/unembedding.py:50-61)."""

    def __init__(self, n_embd, vocab_size, padded_vocab_size, norm, softcap=None):
        super().__init__()
        self.vocab_size = vocab_size
        self.norm = norm
        self.softcap = softcap
        self.lm_head = Linear(n_embd, padded_vocab_size, bias=False)

    @torch.no_grad()
    def init_weights(self):
        nn.init.normal_(self.lm_head.weight, mean=0.0, std=0.001)

    def forward(self, x, h=None):
        """h, when given, is norm(x) already made by the last block."""
        logits = self.lm_head(self.norm(x) if h is None else h)[..., :self.vocab_size].float()
        if self.softcap is not None:
            logits = self.softcap * torch.tanh(logits / self.softcap)
        return logits


# -----------------------------------------------------------------------------------------------
# Model
# -----------------------------------------------------------------------------------------------
def _default_attention():
    from modelcore_amd.kernels.flash_attn import flash_attn
    return flash_attn


def _default_epilogue():
    from modelcore_amd.kernels.qk_epilogue import rope_norm_scale_append
    return rope_norm_scale_append


class Model(nn.Module):
    """Embedding -> blocks -> lm_head; advances the cache once per forward, after every layer
    (modelcore/model.py:93-101)."""

    def __init__(self, config: ModelConfig, runtime: Runtime | None = None, attention=None,
                 epilogue=None):
        super().__init__()
        self.config = config
        self.runtime = runtime or Runtime()
        if attention is None:  # the native operator, and with it the fused pre-attention step
            attention = _default_attention()
            epilogue = epilogue or _default_epilogue()
        shared = {}
        for name, spec in config.shared.items():
            if spec.type == "rotary":
                shared[name] = Rotary(spec.params["head_dim"], config.sequence_len,
                                      spec.params.get("over_compute", 10), self.runtime)
            elif spec.type == "rms_norm":
                shared[name] = RMSNorm(spec.params.get("eps"))
            else:
                raise NotImplementedError(f"shared component {spec.type!r} is not supported")
        self.shared = nn.ModuleDict(shared)
        rope, norm = shared["rope"], shared["norm"]

        inp = config.input
        assert inp.type == "token_embedding", inp.type
        self.embedding = TokenEmbedding(config.padded_vocab_size, config.n_embd, norm,
                                        self.runtime, smear=inp.params.get("smear", False))
        body = config.body
        assert body.type == "stack", body.type
        if body.params.get("features"):
            raise NotImplementedError("stack features are not supported")
        blocks = []
        for spec in body.params["blocks"]:
            assert spec.type == "block", spec.type
            p = spec.params
            if p.get("features"):
                raise NotImplementedError("block features are not supported")
            m = p["mixer"]
            assert m.type == "attention", f"mixer {m.type!r} is not supported"
            mp = m.params
            mixer = Attention(config.n_embd, mp["n_head"], mp.get("n_kv_head", mp["n_head"]),
                              mp.get("head_dim"), mp.get("window", -1), mp.get("kv_slot"),
                              mp.get("produces_kv", True), mp.get("features"), rope, norm,
                              attention, epilogue)
            f = p["ffn"]
            ffn_cls = {"gated_mlp": GatedMLP, "mlp": MLP}[f.type]
            ffn = ffn_cls(config.n_embd, f.params["activation"], f.params["hidden_dim"])
            blocks.append(Block(p["layer_idx"], mixer, ffn, norm))
        self.body = Stack(blocks)
        out = config.output
        assert out.type == "lm_head", out.type
        self.unembedding = LMHead(config.n_embd, config.vocab_size, config.padded_vocab_size, norm,
                                  out.params.get("softcap"))

    @torch.no_grad()
    def init_weights(self):
        """RNG draws in the reference's order: embedding, shared, blocks in order (attention then
        ffn), lm_head (modelcore/model.py:63-69)."""
        self.embedding.init_weights()
        for m in self.shared.values():
            m.init_weights()
        self.body.init_weights()
        self.unembedding.init_weights()

    @torch.no_grad()
    def cache_inference_weights(self, dtype=None, fuse=True):
        """Keep a copy of every Linear weight in `dtype` (default: the compute dtype) and use it
        instead of casting the fp32 master weight at every call: the per-step weight traffic of a
        decode drops from a read of the fp32 weights plus a write and a read of the cast copy to
        one read of the copy. With ``fuse=False`` the products are bit-identical to the uncached
        ones (the cast is the same). With ``fuse`` (the default) the copies of W_q, W_k, W_v of
        each KV-producing attention layer, and of W_gate, W_up of each gated MLP, are stacked so
        one product reads each group in one pass -- the same dot products, which the library GEMM
        may sum in another order (differences at the rounding of the compute dtype). Call again
        after the master weights change; ``drop_inference_weights`` undoes it."""
        dtype = dtype or self.runtime.compute_dtype
        self.drop_inference_weights()
        for m in self.modules():
            if fuse and isinstance(m, Attention) and m.produces_kv:
                stacked = torch.cat([m.c_q.weight, m.c_k.weight, m.c_v.weight]).to(dtype)
                m._qkv = stacked
                q, kv = m.c_q.out_features, m.c_k.out_features
                m.c_q._cast, m.c_k._cast, m.c_v._cast = stacked.split([q, kv, kv])
            elif fuse and isinstance(m, GatedMLP):
                from modelcore_amd.kernels.linear import GATE_BLOCK, interleave_gate_up
                if m.hidden_dim % GATE_BLOCK == 0:
                    # Gate and up rows interleaved in blocks of 64, the layout of the fused
                    # SiLU-product kernel; the separate gate/up rows have no view of their own.
                    m._gate_up = interleave_gate_up(m.gate_proj.weight, m.up_proj.weight).to(dtype)
                    m._gate_up_blocked = True
                    m.gate_proj._in_stack = m.up_proj._in_stack = True
                else:
                    stacked = torch.cat([m.gate_proj.weight, m.up_proj.weight]).to(dtype)
                    m._gate_up = stacked
                    m.gate_proj._cast, m.up_proj._cast = stacked.split(m.hidden_dim)
        for m in self.modules():
            if isinstance(m, Linear) and m._cast is None and not m._in_stack:
                m._cast = m.weight.detach().to(dtype)
        if any(isinstance(m, Linear) and m.skinny for m in self.modules()):
            self.use_skinny_gemm(True)  # the stacks' layout for the skinny GEMM

    def drop_inference_weights(self):
        for m in self.modules():
            if isinstance(m, Linear):
                m._cast = None
                m._in_stack = False
            elif isinstance(m, Attention):
                m._qkv = None
            elif isinstance(m, GatedMLP):
                m._gate_up = None
                m._gate_up_blocked = False

    def set_fused_residual(self, enabled: bool):
        """Run each block's residual adds and the RMS-norms after them as one launch each
        (residual_rmsnorm), with the norm carried into the next block and the lm_head, and let
        c_proj / down_proj hand over their unsummed K-split partials when they run on the skinny
        GEMM (and the stacked QKV product its partials to the fused pre-attention step, which
        sums them). For bf16 decode-sized rows; results differ from the separate ops only in the
        order of the norm's fp32 sum of squares. Needs the parameterless RMSNorm."""
        if enabled and not isinstance(self.shared["norm"], RMSNorm):
            raise NotImplementedError("fused residual steps need the rms_norm shared norm")
        for block in self.body.blocks:
            block.fuse_residual = bool(enabled)
            block.mixer.qkv_partial = bool(enabled)
            block.mixer.c_proj.partial = bool(enabled)
            out = getattr(block.ffn, "down_proj", None) or block.ffn.c_proj
            out.partial = bool(enabled)

    def use_skinny_gemm(self, enabled: bool):
        """Run the projections of decode-sized batches (at most 64 rows, bf16 cached weights)
        through ``mcamd_linear_bf16`` instead of F.linear; other shapes keep F.linear. The
        interleaved gate/up stacks are kept tiled while it is on (``linear.tile_weight``: the
        gated product then streams whole 1 KB runs of them), row-major while it is off; a library
        product on a tiled stack (a prefill) reads a row-major copy."""
        from modelcore_amd.kernels import linear as lin
        for m in self.modules():
            if isinstance(m, Linear):
                m.skinny = bool(enabled)
            elif isinstance(m, GatedMLP) and m._gate_up_blocked:
                tiled = m._gate_up.dim() == 4
                if enabled and not tiled:
                    m._gate_up = lin.tile_weight(m._gate_up)
                elif not enabled and tiled:
                    m._gate_up = lin.untile_weight(m._gate_up)

    def set_fused_epilogue(self, enabled: bool):
        """Choose, for every attention layer at once, between the fused pre-attention launch
        (RoPE + QK-norm + x1.2 + append; the default with the native operator) and the
        reference's separate ops. Results agree within one unit in the last place."""
        for b in self.body.blocks:
            b.mixer.fuse_epilogue = bool(enabled)

    def layer_specs(self):
        return [b.mixer.layer_spec() for b in self.body.blocks]

    def get_device(self):
        return next(self.parameters()).device

    @staticmethod
    def check_cache_room(kv_cache, T):
        """T more positions must fit in the cache: the reference fails at the cache write
        (an index error past T_max), which the kernels cannot raise, so the check is made here
        -- free on a uniform cache (the host mirror), one host read on a ragged one (as the
        ragged RoPE gather makes anyway)."""
        if isinstance(kv_cache, PackedPrefill):
            # Empty rows and prompt lengths within the cache and the rotary table: checked when
            # the packed batch was made, apart from the table's length.
            assert kv_cache.max_seqlen <= kv_cache.cache.max_seq_len
            return
        pos = kv_cache.uniform_pos()
        last = pos + T if pos is not None else int(kv_cache.cache_seqlens.max().item()) + T
        assert last <= kv_cache.max_seq_len, \
            f"Sequence length {last} exceeds cache length {kv_cache.max_seq_len}"

    def forward(self, idx, targets=None, kv_cache=None):
        if targets is not None:
            raise NotImplementedError("training loss is not part of the inference path")
        if kv_cache is not None:
            self.check_cache_room(kv_cache, idx.size(1))
        x = self.embedding(idx)
        x, h = self.body.forward_carry(x, kv_cache)
        if kv_cache is not None:
            kv_cache.advance(idx.size(1))
        return self.unembedding(x, h)

    def last_logits(self, idx, kv_cache, last):
        """forward(), but the head runs only at position last[b] of row b: (B, vocab) logits.
        The head is per position, so these equal forward()[b, last[b]]; a prompt prefill needs
        only its last position, and skips the (B, T, vocab) logits of all the others. With a
        PackedPrefill, idx is every prompt's tokens as one (1, total) sequence, `last` is not
        used, and the logits are those of each prompt's last token, (prompts, vocab)."""
        self.check_cache_room(kv_cache, idx.size(1))
        if isinstance(kv_cache, PackedPrefill):
            assert idx.size(0) == 1 and idx.size(1) == kv_cache.total, \
                "a packed prefill takes every prompt's tokens as one (1, total) sequence"
            n_pos = min(b.mixer.rope.cos.size(1) for b in self.body.blocks)
            assert kv_cache.max_seqlen <= n_pos, \
                f"Sequence length grew beyond the rotary embeddings cache: {kv_cache.max_seqlen} > {n_pos}"
        x, h = self.body.forward_carry(self.embedding(idx), kv_cache)
        kv_cache.advance(idx.size(1))
        if isinstance(kv_cache, PackedPrefill):  # (prompts, vocab) at each prompt's last token
            last = kv_cache.last
            return self.unembedding(x[0, last].unsqueeze(1),
                                    None if h is None else h[0, last].unsqueeze(1))[:, 0]
        rows = torch.arange(idx.size(0), device=x.device)
        last = last.to(x.device)
        return self.unembedding(x[rows, last].unsqueeze(1),
                                None if h is None else h[rows, last].unsqueeze(1))[:, 0]


def kv_cache_spec(layer_specs):
    """num_kv_slots / n_kv_head / head_dim for KVCache (modelcore/stats.py:110-131): one slot per
    distinct kv_slot, which must form 0..M-1; uniform n_kv_head and head_dim."""
    assert layer_specs, "layer_specs is empty"
    assert len({s.n_kv_head for s in layer_specs}) == 1 and \
        len({s.head_dim for s in layer_specs}) == 1, \
        "kv_cache_spec() requires uniform n_kv_head/head_dim across layers"
    slots = {s.kv_slot for s in layer_specs}
    assert slots == set(range(len(slots))), \
        "kv_cache_spec() requires kv slots to be a contiguous 0..M-1 range"
    return {"n_kv_head": layer_specs[0].n_kv_head, "head_dim": layer_specs[0].head_dim,
            "num_kv_slots": len(slots)}


class ModelManager:
    """create_model / new_kv_cache / new_decoder (modelcore/manager.py:111-119, :286-299)."""

    def __init__(self, runtime: Runtime | None = None, attention=None, epilogue=None):
        self.runtime = runtime or Runtime()
        self.attention = attention
        self.epilogue = epilogue

    def create_model(self, config, *, device, seed=None):
        if isinstance(config, dict):
            config = ModelConfig.from_dict(config)
        with torch.device("meta"):
            model = Model(config, runtime=self.runtime, attention=self.attention,
                          epilogue=self.epilogue)
        model.to_empty(device=device)
        if seed is not None:
            torch.manual_seed(seed)
        model.init_weights()
        return model

    def new_kv_cache(self, model, *, batch_size, seq_len, device=None):
        spec = kv_cache_spec(model.layer_specs())
        return KVCache(batch_size=batch_size, seq_len=seq_len,
                       device=device or model.get_device(), dtype=self.runtime.compute_dtype,
                       **spec)

    def new_decoder(self, model, tokens, *, num_samples=1, max_tokens=None, device=None):
        from modelcore_amd.generate import Decoder
        return Decoder(model, self, tokens, num_samples=num_samples, max_tokens=max_tokens,
                       device=device)


def param_count(model) -> int:
    return sum(p.numel() for p in model.parameters())
