"""``nn.MultiheadAttention`` on the GPU (the reference's module: ``python/densecore/nn.py:595-640``).

The module follows PyTorch's documented ``torch.nn.MultiheadAttention``: its constructor
arguments, its parameters (names, shapes, and which of them exist for a given configuration) and
its initialisation (``_reset_parameters``: xavier-uniform input projections, zero input and
output projection biases, xavier-normal ``bias_k`` / ``bias_v``), with the parameters on the GPU
and the forward through ``functional.multi_head_attention_forward``.  Initial values come from
torch's generator (the reference draws them from its own CPU generator), so two freshly built
modules agree in distribution, not in bits: load the same weights to compare outputs.
"""
import torch

from . import functional


class MultiheadAttention(torch.nn.Module):
    """Multi-head attention (Q, K, V projections, ``num_heads`` heads of ``embed_dim //
    num_heads`` dims, output projection) with PyTorch's parameterisation; forward returns
    ``(attn_output, attn_weights)``, the weights averaged over heads unless asked otherwise."""

    def __init__(self, embed_dim, num_heads, dropout=0.0, bias=True, add_bias_kv=False,
                 add_zero_attn=False, kdim=None, vdim=None, batch_first=False, device=None,
                 dtype=None):
        super().__init__()
        if embed_dim <= 0 or num_heads <= 0:
            raise ValueError("embed_dim and num_heads must be greater than 0")
        if embed_dim % num_heads:
            raise AssertionError("embed_dim must be divisible by num_heads")
        where = {"device": torch.device("cuda") if device is None else torch.device(device),
                 "dtype": torch.float32 if dtype is None else dtype}
        self.embed_dim = embed_dim
        self.num_heads = num_heads
        self.head_dim = embed_dim // num_heads
        self.dropout = dropout
        self.batch_first = batch_first
        self.add_zero_attn = add_zero_attn
        self.kdim = kdim if kdim else embed_dim
        self.vdim = vdim if vdim else embed_dim
        # One packed (3E, E) input projection when keys and values have the query's width.
        self._qkv_same_embed_dim = self.kdim == embed_dim and self.vdim == embed_dim

        def param(*shape):
            return torch.nn.Parameter(torch.empty(shape, **where))

        packed = self._qkv_same_embed_dim
        self.in_proj_weight = param(3 * embed_dim, embed_dim) if packed else None
        self.q_proj_weight = None if packed else param(embed_dim, embed_dim)
        self.k_proj_weight = None if packed else param(embed_dim, self.kdim)
        self.v_proj_weight = None if packed else param(embed_dim, self.vdim)
        self.in_proj_bias = param(3 * embed_dim) if bias else None
        self.out_proj = torch.nn.Linear(embed_dim, embed_dim, bias=bias, **where)
        self.bias_k = param(1, 1, embed_dim) if add_bias_kv else None
        self.bias_v = param(1, 1, embed_dim) if add_bias_kv else None
        self._reset_parameters()

    def _reset_parameters(self):
        """PyTorch's initial values: xavier-uniform input projection weight(s), zero input and
        output projection biases (the output projection's weight keeps ``Linear``'s own
        initialisation), xavier-normal ``bias_k`` and ``bias_v``."""
        init = torch.nn.init
        if self._qkv_same_embed_dim:
            init.xavier_uniform_(self.in_proj_weight)
        else:
            for w in (self.q_proj_weight, self.k_proj_weight, self.v_proj_weight):
                init.xavier_uniform_(w)
        if self.in_proj_bias is not None:
            init.zeros_(self.in_proj_bias)
            init.zeros_(self.out_proj.bias)
        if self.bias_k is not None:
            init.xavier_normal_(self.bias_k)
            init.xavier_normal_(self.bias_v)

    def forward(self, query, key, value, key_padding_mask=None, need_weights=True, attn_mask=None,
                average_attn_weights=True, is_causal=False):
        # batch_first inputs (N, L, E) go through the functional form as (L, N, E) and back.
        swap = self.batch_first and query.dim() == 3
        if swap:
            query, key, value = query.transpose(0, 1), key.transpose(0, 1), value.transpose(0, 1)
        out, weights = functional.multi_head_attention_forward(
            query, key, value, self.embed_dim, self.num_heads, self.in_proj_weight,
            self.in_proj_bias, self.bias_k, self.bias_v, self.add_zero_attn, self.dropout,
            self.out_proj.weight, self.out_proj.bias, training=self.training,
            key_padding_mask=key_padding_mask, need_weights=need_weights, attn_mask=attn_mask,
            use_separate_proj_weight=not self._qkv_same_embed_dim,
            q_proj_weight=self.q_proj_weight, k_proj_weight=self.k_proj_weight,
            v_proj_weight=self.v_proj_weight, average_attn_weights=average_attn_weights,
            is_causal=is_causal)
        return (out.transpose(0, 1) if swap else out), weights
