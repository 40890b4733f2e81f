"""HIP payload codec at K1..K6 against the host codec, and the uniform-rate
encode entry point at K2, K5 and K6: closed payload at exactly K bits per
weight that decodes to the reported reconstruction."""

from __future__ import annotations

import sys

import pytest
import torch

from qsrt_amd.codec import pack_words, unpack_words
from qsrt_amd.exl3_reference import decode_exl3_weight
from qsrt_amd.qsrt_codec_pilot import encode_uniform_candidate, replay_uniform_candidate, unpack_uniform_trellis_states
from qsrt_amd.sqg_e4m3 import sqg_codebook

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda:0")


@pytest.mark.parametrize("bits", [1, 2, 3, 4, 5, 6])
def test_hip_codec_matches_host(bits):
    print(f"[codec] K{bits}", file=sys.stderr, flush=True)
    g = torch.Generator().manual_seed(40 + bits)
    states = torch.randint(-32768, 32768, (37, 256), generator=g).to(torch.int16)
    words = pack_words(states.to(DEV), bits).cpu()
    assert torch.equal(words, pack_words(states, bits))
    assert torch.equal(unpack_words(words.to(DEV), bits).cpu(), unpack_words(words, bits))


@pytest.mark.parametrize("bits", [2, 5, 6])
def test_encode_uniform_candidate(bits):
    print(f"[codec] encode_uniform_candidate K{bits} 256x128", file=sys.stderr, flush=True)
    g = torch.Generator().manual_seed(bits)
    source = 0.02 * torch.randn(256, 128, generator=g)   # [out, in]
    x = torch.randn(2048, 128, generator=g)
    h = x.T @ x / 2048
    res = encode_uniform_candidate(source, bits=bits, codebook="sqg_xor_cheb_t12", device=DEV, input_sign_seed=11,
                                   output_sign_seed=12, hessian=h, return_replay_state=True)
    pay = res["payload"]
    assert pay["rate"] == bits and pay["trellis_bpw"] == float(bits)
    assert pay["input_hessian_role"] == "caller_supplied_curvature"
    assert 0.0 < pay["proxy_relative_error"] < 0.5
    rec = res["reconstruction"]
    assert rec.shape == source.shape and rec.dtype == torch.float16
    err = float((rec.float() - source).norm() / source.norm())
    assert err < {2: 0.5, 5: 0.1, 6: 0.06}[bits], err
    state = res["replay_state"]

    def decode_on(device):
        states = unpack_uniform_trellis_states(state["trellis"].to(device), bits)
        return decode_exl3_weight(states, state["suh"].to(device), state["svh"].to(device),
                                  codebook="sqg_xor_cheb_t12", bits=bits).half().T.contiguous().cpu()

    assert torch.equal(decode_on(DEV), rec)  # the payload decodes to the reported reconstruction
    host = decode_on("cpu")                  # host and device Hadamards round differently in fp16
    assert float((host.float() - rec.float()).abs().max() / rec.float().abs().max()) < 2e-3
    table = sqg_codebook(bits, "sqg_xor_cheb_t12", dtype=torch.float16)
    assert torch.equal(replay_uniform_candidate(state, codebook_values=table), host)
