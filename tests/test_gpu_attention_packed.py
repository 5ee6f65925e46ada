"""GPU parity of the spike self-attention path on packed spikes.

Packed q/k/v put every head on whole 32-bit words (``slot`` bits, the bits
past d zero).  The packed core must give the integer counts Q K^T and
(Q K^T) V of the oracle bit for bit and exactly the spikes of the bf16 core;
the packed SSA block the same Q/K/V and attention spikes as the bf16 block
and its output within fp32-summation tolerance (the head padding changes
only the grouping of the output projection's sums).
"""
import pytest
import torch

from oracle import neurons as on
from snnk.kernels.binary import pack_bits
from snnk.kernels.attention import (spike_attention, spike_attention_packed, spike_self_attention,
                                    spike_self_attention_packed, prepare_ssa_packed)
from snnk.kernels.linear import linear_preact, linear_preact_act

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _spikes(shape, p, seed):
    return (torch.rand(*shape, generator=torch.Generator().manual_seed(seed)) < p).float()


def _pack_heads(x, heads, slot):
    """spikes [T, R, heads*d] -> int32 words [T, R, heads*slot/32], each head
    padded with zeros to ``slot`` bits."""
    T, R, HD = x.shape
    d = HD // heads
    xp = torch.zeros(T, R, heads, slot, device=x.device, dtype=x.dtype)
    xp[..., :d] = x.view(T, R, heads, d)
    return pack_bits(xp.reshape(T, R, heads * slot), dim=-1)


def _unpack_heads(words, heads, slot, d):
    """int32 words -> 0/1 [T, R, heads*d]; asserts the padding bits are zero."""
    bits = (words.unsqueeze(-1) >> torch.arange(32, device=words.device)) & 1
    T, R = words.shape[:2]
    b = bits.reshape(T, R, heads, slot)
    assert not bool(b[..., d:].any()), "bits past d must be zero"
    return b[..., :d].reshape(T, R, heads * d).float()


@pytest.mark.parametrize("T,B,H,N,d,soft,v_reset", [
    (4, 32, 8, 64, 48, False, 0.0), (4, 2, 4, 64, 8, False, 0.0), (3, 3, 2, 49, 64, True, 0.0),
    (1, 2, 3, 16, 32, False, 0.25), (5, 1, 1, 33, 40, True, 0.0), (4, 4, 6, 64, 16, False, -0.5)])
def test_packed_core_counts_and_spikes_exact(T, B, H, N, d, soft, v_reset):
    D = H * d
    slot = 32 * ((d + 31) // 32)
    qkv = _spikes((T, B * N, 3 * D), 0.25, N + d + 7)
    qd = qkv.to(DEV, torch.bfloat16)
    q, k, v = qd[..., :D], qd[..., D:2 * D], qd[..., 2 * D:]
    kw = dict(B=B, N=N, heads=H, scale=0.125, tau=2.0, v_threshold=0.5, v_reset=v_reset,
              soft_reset=soft, return_counts=True)
    ref, S_ref, O_ref = spike_attention(q, k, v, **kw)
    Hw = H * slot // 32
    # heads back to back (as a packed projection writes them; D % 32 == 0
    # needed for one packed row of q|k|v) and heads padded to whole words
    layouts = [("padded", torch.cat([_pack_heads(t, H, slot) for t in (q, k, v)], -1), slot, Hw)]
    if D % 32 == 0:
        layouts.append(("back to back", pack_bits(qd, dim=-1), d, D // 32))
    for name, words, hbits, wq in layouts:
        words = words.contiguous()
        got, S, O = spike_attention_packed(words[..., :wq], words[..., wq:2 * wq], words[..., 2 * wq:],
                                           d=d, in_head_bits=hbits, out_head_words=slot // 32, **kw)
        assert got.shape == (T, B * N, Hw) and got.dtype == torch.int32, name
        assert torch.equal(S, S_ref) and torch.equal(O, O_ref), name
        assert torch.equal(_unpack_heads(got, H, slot, d), ref.float()), name
    # and the oracle's LIF on the exact counts
    hq = lambda s: s.view(T, B, N, H, d).permute(0, 1, 3, 2, 4).long()  # noqa: E731
    O_cpu = (hq(qkv[..., :D]) @ hq(qkv[..., D:2 * D]).transpose(-1, -2)) @ hq(qkv[..., 2 * D:])
    assert torch.equal(O.cpu().long(), O_cpu)
    a_ref, _, _ = on.lif_multistep(O_cpu.float() * 0.125, neuron="lif", tau=2.0, soft_reset=soft,
                                   v_threshold=0.5, v_reset=v_reset)
    assert torch.equal(_unpack_heads(got, H, slot, d).cpu().view(T, B, N, H, d).permute(0, 1, 3, 2, 4),
                       a_ref)


def test_packed_core_rejects_what_it_does_not_cover():
    from snnk._abi import SnnkError
    w = torch.zeros(1, 4 * 65, 9, device=DEV, dtype=torch.int32)
    with pytest.raises(SnnkError):          # more than 64 tokens: no packed linear order
        spike_attention_packed(w[..., :3], w[..., 3:6], w[..., 6:9], B=4, N=65, heads=1,
                               d=72, in_head_bits=72, out_head_words=3, scale=0.125)
    with pytest.raises(SnnkError):          # output slot too small for d
        spike_attention_packed(w[:, :64, :2], w[:, :64, 2:4], w[:, :64, 4:6], B=1, N=64, heads=1,
                               d=48, in_head_bits=48, out_head_words=1, scale=0.125)
    with pytest.raises(SnnkError):          # head bit stride not a multiple of 8
        spike_attention_packed(w[:, :64, :2], w[:, :64, 2:4], w[:, :64, 4:6], B=1, N=64, heads=1,
                               d=40, in_head_bits=44, out_head_words=2, scale=0.125)


def test_linear_preact_act_packed_matches_bf16():
    g = torch.Generator().manual_seed(5)
    T, R, K, N = 4, 64, 512, 384
    x = _spikes((T, R, K), 0.3, 6).to(DEV, torch.bfloat16)
    w = (torch.randn(N, K, generator=g) * K ** -0.5).to(DEV, torch.bfloat16)
    b = (torch.randn(N, generator=g) * 0.1).to(DEV)
    ref = linear_preact(x.contiguous(), w, b)
    got = linear_preact_act(pack_bits(x, dim=-1), w, b)
    assert torch.equal(got, ref)     # same kernel tiles and K order: identical sums
    got_bf = linear_preact_act(x.contiguous(), w, b)
    assert torch.equal(got_bf, ref)


@pytest.mark.parametrize("T,B,N,D,H", [(4, 32, 64, 384, 8), (2, 4, 33, 256, 4), (3, 2, 64, 192, 3)])
def test_packed_ssa_block_matches_bf16_block(T, B, N, D, H):
    g = torch.Generator().manual_seed(T * 100 + D)
    x = _spikes((T, B, N, D), 0.2, D + N)
    w_qkv = (torch.randn(3 * D, D, generator=g) * (2.0 / D) ** 0.5).to(DEV, torch.bfloat16)
    b_qkv = (torch.randn(3 * D, generator=g) * 0.1).to(DEV)
    w_p = (torch.randn(D, D, generator=g) * (2.0 / D) ** 0.5).to(DEV, torch.bfloat16)
    b_p = (torch.randn(D, generator=g) * 0.1).to(DEV)
    ref, inter = spike_self_attention(x.to(DEV), w_qkv, b_qkv, w_p, b_p, heads=H,
                                      return_intermediates=True)
    prep = prepare_ssa_packed(w_qkv, b_qkv, w_p, heads=H)
    xw = pack_bits(x.to(DEV).reshape(T, B * N, D), dim=-1)
    got, pi = spike_self_attention_packed(xw, prep, b_p, B=B, N=N, return_intermediates=True)
    d, slot = D // H, prep["slot"]
    qkv_bits = (pi["qkv"].unsqueeze(-1) >> torch.arange(32, device=DEV)) & 1
    assert torch.equal(qkv_bits.reshape(T, B * N, 3 * D).float(), inter["qkv"].float())
    assert torch.equal(_unpack_heads(pi["attn"], H, slot, d), inter["attn"].float())
    assert torch.equal(pi["O"], inter["O"])
    scale = ref.abs().max().item()
    assert (got - ref).abs().max().item() <= 1e-5 * max(1.0, scale) * 4
