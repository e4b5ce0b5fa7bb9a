"""The MoE decoder around the MoE layer (no GPU compute): parameter layout, init RNG order,
and the torch-side pieces against closed forms (reference: abacus/transformer_moe.py:17-75,
transformer_block.py:64-110, attention.py:67-150, rope.py:9-46, norm.py:11-31, embedding.py:8-23)."""

import math

import pytest
import torch

from abacus.attention import MultiHeadAttention
from abacus.embedding import Embedding
from abacus.moe.moe import MoE
from abacus.norm import RMSNorm
from abacus.rope import Rotary, apply_rotary_pos_emb, rotate_half
from abacus.transformer_block import TransformerBlockMoe
from abacus.transformer_moe import TransformerMoe
from abacus_amd.transformer import _CausalAttention

CFG = dict(dim=32, n_heads=4, head_dim=8, n_blocks=2, vocab_size=50, n_experts=4, top_k=2, hidden_dim=48)


def test_state_dict_layout():
    m = TransformerMoe(**CFG)
    shapes = {k: tuple(v.shape) for k, v in m.state_dict().items()}
    D, H, K, V, E, M = 32, 4, 8, 50, 4, 48
    want = {"w_D_vocab": (D, V), "embedding.w_vocab_D": (V, D), "rotary.inv_freq": (K // 2,), "norm.w_gamma_D": (D,)}
    for b in range(2):
        p = f"blocks.{b}."
        want.update({
            p + "norm_attention.w_gamma_D": (D,), p + "norm_mlp.w_gamma_D": (D,),
            p + "attention.w_q_DHK": (D, H, K), p + "attention.w_k_DHK": (D, H, K), p + "attention.w_v_DHK": (D, H, K),
            p + "attention.w_o_HKD": (H, K, D), p + "attention.q_norm.w_gamma_D": (K,),
            p + "attention.k_norm.w_gamma_D": (K,),
            p + "moe.router.w_DE": (D, E), p + "moe.router.expert_bias_E": (E,),
            p + "moe.w_gate_EDM": (E, D, M), p + "moe.w_up_EDM": (E, D, M), p + "moe.w_down_EMD": (E, M, D),
        })
    assert shapes == want


def test_init_rng_order_matches_reference_sequence():
    """Replays the reference constructors' RNG draws in order (transformer_moe.py:43-64)."""
    torch.manual_seed(123)
    m = TransformerMoe(**CFG)
    D, H, K, V = 32, 4, 8, 50
    torch.manual_seed(123)
    emb = torch.empty(V, D).normal_()  # embedding.py:16-17
    blocks = []
    for _ in range(2):
        qkv = []
        for _ in range(3):  # attention.py:99-105: q, k, v on their (D, H*K) views
            w = torch.empty(D, H, K)
            torch.nn.init.xavier_uniform_(w.view(D, H * K))
            qkv.append(w)
        o = torch.empty(H, K, D)
        torch.nn.init.xavier_uniform_(o.view(H * K, D))  # attention.py:106
        moe = MoE(D, 4, 2, hidden_dim=48)  # its own RNG order is pinned in test_api.py
        blocks.append((qkv, o, moe))
    w_vocab = torch.empty(D, V)
    torch.nn.init.xavier_uniform_(w_vocab)  # transformer_moe.py:63-64
    assert torch.equal(m.embedding.w_vocab_D, emb)
    assert torch.equal(m.w_D_vocab, w_vocab)
    for blk, (qkv, o, moe) in zip(m.blocks, blocks):
        a = blk.attention
        for got, want in zip((a.w_q_DHK, a.w_k_DHK, a.w_v_DHK), qkv):
            assert torch.equal(got, want)
        assert torch.equal(a.w_o_HKD, o)
        for name, t in moe.state_dict().items():
            assert torch.equal(blk.moe.state_dict()[name], t), name


def test_causal_attention_gradcheck():
    g = torch.Generator().manual_seed(0)
    q, k, v = (torch.randn(3, 5, 4, generator=g, dtype=torch.float64, requires_grad=True) for _ in range(3))
    assert torch.autograd.gradcheck(lambda a, b, c: _CausalAttention.apply(a, b, c, 2.0), (q, k, v))


def test_attention_matches_plain_restatement():
    torch.manual_seed(1)
    mha = MultiHeadAttention(32, 4, 8).double()
    rot = Rotary(8).double()
    x = torch.randn(2, 7, 32, dtype=torch.float64)
    got = mha(x, rot)
    # attention.py:129-145 written with einsum and masked softmax
    def split(w):
        return (x @ w.reshape(32, 32)).view(2, 7, 4, 8).permute(0, 2, 1, 3)
    q, k, v = split(mha.w_q_DHK), split(mha.w_k_DHK), split(mha.w_v_DHK)
    q, k = mha.q_norm(q), mha.k_norm(k)
    cos, sin = rot(q)
    q, k = apply_rotary_pos_emb(q, k, cos, sin)
    s = torch.einsum("bhlk,bhsk->bhls", q, k) / math.sqrt(8)
    pos = torch.arange(7)
    s = s.masked_fill(pos[:, None] < pos[None, :], float("-inf"))
    o = torch.einsum("bhls,bhsk->bhlk", torch.softmax(s, -1), v)
    want = o.permute(0, 2, 1, 3).reshape(2, 7, 32) @ mha.w_o_HKD.reshape(32, 32)
    torch.testing.assert_close(got, want, rtol=1e-12, atol=1e-12)


def test_rotary_and_rmsnorm_closed_forms():
    rot = Rotary(4, base=100.0)
    x = torch.zeros(1, 1, 3, 4)
    cos, sin = rot(x)
    inv = torch.tensor([1.0, 0.1])
    ang = torch.arange(3.0)[:, None] * torch.cat([inv, inv])[None, :]
    torch.testing.assert_close(cos[0, 0], ang.cos())
    torch.testing.assert_close(sin[0, 0], ang.sin())
    assert torch.equal(rotate_half(torch.tensor([1.0, 2.0, 3.0, 4.0])), torch.tensor([-3.0, -4.0, 1.0, 2.0]))
    n = RMSNorm(3)
    y = n(torch.tensor([[3.0, 0.0, 4.0]]))
    torch.testing.assert_close(y, torch.tensor([[3.0, 0.0, 4.0]]) / math.sqrt(25 / 3 + 1e-5))
    e = Embedding(10, 3)
    assert torch.equal(e(torch.tensor([[2, 7]])), e.w_vocab_D[[2, 7]].unsqueeze(0))


def test_constructor_errors():
    with pytest.raises(ValueError, match="sequence_parallel requires tensor_parallel"):
        MultiHeadAttention(8, 2, 4, sequence_parallel=True)
    with pytest.raises(ValueError, match="does not combine"):
        MultiHeadAttention(8, 2, 4, tensor_parallel=True, context_parallel=True)
    blk = TransformerBlockMoe(16, 2, 8, 4, 2, dropout=0.1, expert_parallel=True)  # one process: allowed
    assert blk.moe.__class__.__name__ == "MoEExpertParallel"
