"""``nn.MultiheadAttention`` on the GPU (``python/densecore/nn.py:595-640`` of the reference).

Same constructor arguments, parameter names and shapes, initialisation rules (xavier-uniform
projection weights, zero projection biases, zero ``out_proj.bias``, xavier-normal ``bias_k`` /
``bias_v``) and forward as the reference module; the parameters live on the GPU and the forward
is ``functional.multi_head_attention_forward``.  Initial values come from torch's generator
(the reference draws them from its own CPU generator), so two freshly built modules agree in
distribution, not in bits: load the same weights to compare outputs.
"""
import torch

from . import functional


class MultiheadAttention(torch.nn.Module):
    """torch.nn.MultiheadAttention: same parameters, initialization and forward."""

    def __init__(self, embed_dim, num_heads, dropout=0.0, bias=True, add_bias_kv=False,
                 add_zero_attn=False, kdim=None, vdim=None, batch_first=False, device=None,
                 dtype=None):
        super().__init__()
        if embed_dim <= 0 or num_heads <= 0:
            raise ValueError("embed_dim and num_heads must be greater than 0")
        if embed_dim % num_heads:
            raise AssertionError("embed_dim must be divisible by num_heads")
        device = torch.device("cuda") if device is None else torch.device(device)
        dtype = torch.float32 if dtype is None else dtype
        self.embed_dim, self.num_heads, self.dropout = embed_dim, num_heads, dropout
        self.batch_first = batch_first
        self.kdim, self.vdim = kdim or embed_dim, vdim or embed_dim
        self._qkv_same_embed_dim = self.kdim == embed_dim and self.vdim == embed_dim
        self.head_dim, self.add_zero_attn = embed_dim // num_heads, add_zero_attn

        def empty(*shape):
            return torch.nn.Parameter(torch.zeros(shape, device=device, dtype=dtype))

        if self._qkv_same_embed_dim:
            self.in_proj_weight = empty(3 * embed_dim, embed_dim)
            self.q_proj_weight = self.k_proj_weight = self.v_proj_weight = None
        else:
            self.q_proj_weight = empty(embed_dim, embed_dim)
            self.k_proj_weight = empty(embed_dim, self.kdim)
            self.v_proj_weight = empty(embed_dim, self.vdim)
            self.in_proj_weight = None
        self.in_proj_bias = empty(3 * embed_dim) if bias else None
        self.out_proj = torch.nn.Linear(embed_dim, embed_dim, bias=bias, device=device, dtype=dtype)
        self.bias_k, self.bias_v = ((empty(1, 1, embed_dim), empty(1, 1, embed_dim)) if add_bias_kv
                                    else (None, None))
        for weight in (self.in_proj_weight, self.q_proj_weight, self.k_proj_weight, self.v_proj_weight):
            if weight is not None:
                torch.nn.init.xavier_uniform_(weight)
        if bias:
            torch.nn.init.zeros_(self.out_proj.bias)
        for extra in (self.bias_k, self.bias_v):
            if extra is not None:
                torch.nn.init.xavier_normal_(extra)

    def forward(self, query, key, value, key_padding_mask=None, need_weights=True, attn_mask=None,
                average_attn_weights=True, is_causal=False):
        batched = query.dim() == 3
        if self.batch_first and batched:
            query, key, value = (x.transpose(1, 0) for x in (query, key, value))
        out, weights = functional.multi_head_attention_forward(
            query, key, value, self.embed_dim, self.num_heads, self.in_proj_weight, self.in_proj_bias,
            self.bias_k, self.bias_v, self.add_zero_attn, self.dropout, self.out_proj.weight,
            self.out_proj.bias, training=self.training, key_padding_mask=key_padding_mask,
            need_weights=need_weights, attn_mask=attn_mask,
            use_separate_proj_weight=not self._qkv_same_embed_dim, q_proj_weight=self.q_proj_weight,
            k_proj_weight=self.k_proj_weight, v_proj_weight=self.v_proj_weight,
            average_attn_weights=average_attn_weights, is_causal=is_causal)
        return (out.transpose(1, 0) if self.batch_first and batched else out), weights
