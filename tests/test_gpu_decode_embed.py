"""GPU parity of tg_decode_embed (the decode step's input rows, model.py:89-90)
through the C ABI.

Bar: the same bf16 bits as torch's `embed[tok] + pos.index_select(0, t)` on the
same device.  Also checked: a token or a position outside its table reads a
zero row (no fault), and int32 or host token ids are accepted.
"""
import pytest
import torch

import decode

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("B,V,P,d,t", [(1, 50257, 1024, 2304, 150), (8, 50257, 1024, 2304, 0),
                                       (3, 512, 64, 256, 63), (2, 100, 10, 8, 9)])
def test_decode_embed_same_bits_as_torch(dev, B, V, P, d, t):
    g = torch.Generator(device=dev).manual_seed(V + d + t)
    embed = torch.randn((V, d), generator=g, device=dev).to(torch.bfloat16)
    pos = (torch.randn((P, d), generator=g, device=dev) * 0.3).to(torch.bfloat16)
    tok = torch.randint(0, V, (B,), generator=g, device=dev)
    tt = torch.tensor([t], dtype=torch.long, device=dev)
    got = decode.decode_embed(embed, pos, tok, tt)
    want = embed[tok] + pos.index_select(0, tt)
    torch.cuda.synchronize()
    assert got.shape == (B, d) and torch.equal(got.view(torch.int16), want.view(torch.int16))
    got32 = decode.decode_embed(embed, pos, tok.to(torch.int32).cpu(), tt)
    assert torch.equal(got32.view(torch.int16), want.view(torch.int16))


def test_decode_embed_outside_the_tables_reads_zero_rows(dev):
    V, P, d = 16, 4, 64
    embed = torch.randn((V, d), device=dev).to(torch.bfloat16)
    pos = torch.randn((P, d), device=dev).to(torch.bfloat16)
    tok = torch.tensor([3, V, -1], dtype=torch.long, device=dev)
    got = decode.decode_embed(embed, pos, tok, torch.tensor([2], dtype=torch.long, device=dev))
    want = torch.stack([embed[3] + pos[2], pos[2], pos[2]])
    assert torch.equal(got.view(torch.int16), want.view(torch.int16))
    got = decode.decode_embed(embed, pos, tok[:1], torch.tensor([P], dtype=torch.long, device=dev))
    assert torch.equal(got.view(torch.int16), embed[3:4].view(torch.int16))
