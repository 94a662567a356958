"""The PyTorch-CPU restatement (oracle/torch_cpu.py, the bench's CPU baseline)
pinned against the C oracle on the bench's input families: INT8 codes, scales
and fp16 outputs and FP8 codes bit for bit; FP8 outputs within 1e-2 of the
float64 recompute; entropies within f32 rounding of the float64 oracle and
probabilities within one fp16 ulp.  (Rows with a zero or non-finite maximum
are outside the restatement, as outside the bench's data.)"""
import numpy as np
import pytest
import torch

import oracle
from oracle import torch_cpu as tc


@pytest.fixture(scope="module")
def data():
    rng = np.random.default_rng(7)
    A = rng.standard_normal((96, 640)).astype(np.float16)
    A[3] *= np.float16(30.0)                         # a large-amax row
    A[5, :] = np.float16(0.5)                        # a constant row
    W = (rng.standard_normal((136, 640)) * 0.02).astype(np.float16)
    B, bs = oracle.quantize_weights_int8(W)          # [K, N] int8, f32 [N]
    s = rng.choice(np.float32([0.25, 1.0, 4.0, 16.0]), 64)
    L = (rng.standard_normal((64, 1000)) * s[:, None]).astype(np.float16)
    return A, B, bs, L


def test_int8_path_bit_exact(data):
    A, B, bs, _ = data
    codes, s = tc.quant_act_i8(torch.from_numpy(A))
    oc, os_ = oracle.quant_act_i8(A, "dispatcher")
    assert np.array_equal(codes.numpy(), oc)
    assert np.array_equal(s.numpy().view(np.uint32), os_.view(np.uint32))
    out = tc.triton_int8_gemm(torch.from_numpy(A), torch.from_numpy(B), torch.from_numpy(bs))
    assert np.array_equal(out.numpy().view(np.uint16), oracle.triton_int8_gemm(A, B, bs).view(np.uint16))


def test_fp8_codes_bit_exact_and_output_close(data):
    A, B, bs, _ = data
    a8, s = tc.quant_act_f8(torch.from_numpy(A))
    oc, os_ = oracle.quant_act_f8(A)
    assert np.array_equal(a8.view(torch.uint8).numpy(), oc)
    assert np.array_equal(s.numpy().view(np.uint32), os_.view(np.uint32))
    w8 = tc.weight_f8(torch.from_numpy(B))
    assert np.array_equal(w8.view(torch.uint8).numpy(), oracle.e4m3_from_f32(B.astype(np.float32)))
    out = tc.triton_fp8_gemm(torch.from_numpy(A), torch.from_numpy(B), torch.from_numpy(bs)).numpy()
    ref = oracle.triton_fp8_gemm_f64(A, B, bs)
    rms = np.sqrt(np.mean(ref ** 2))
    assert (np.abs(out.astype(np.float64) - ref) <= 1e-2 * np.abs(ref) + 1e-3 * rms).all()


def test_softmax_entropy_close(data):
    *_, L = data
    p, h = tc.softmax_entropy(torch.from_numpy(L))
    H, P = oracle.softmax_entropy(L)
    assert np.allclose(h.numpy().astype(np.float64), H, rtol=1e-4, atol=1e-5)
    d = np.abs(p.numpy().view(np.uint16).astype(np.int32) - P.view(np.uint16).astype(np.int32))
    assert d.max() <= 1
