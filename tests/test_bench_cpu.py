"""Host-side contract of bench.py: the refusals, and the byte counts its
roofline figures divide by (no GPU needed)."""

import pytest
import torch

import bench
import mlx_batch_invariant_amd as bi


def test_more_than_one_gpu_is_refused(capsys):
    assert bench.main(["--gpus", "2"]) == 2
    assert "one GPU" in capsys.readouterr().err


@pytest.mark.skipif(torch.cuda.is_available(), reason="checks the no-GPU refusal")
def test_no_gpu_is_refused(capsys):
    assert bench.main([]) == 2
    assert "needs a GPU" in capsys.readouterr().err


@pytest.mark.parametrize("bits,gs", [(4, 64), (8, 128), (4, 32)])
@pytest.mark.parametrize("M", [1, 3])
def test_qmm_bytes_counts_every_tensor_once(bits, gs, M):
    # Independent count: the sizes of the tensors the quantizer actually packs,
    # plus x read once and out written once.
    N, K = 64, 512
    W = torch.randn((N, K), generator=torch.Generator().manual_seed(1))
    wq, s, b = bi.quantize(W, group_size=gs, bits=bits, dtype=torch.bfloat16)
    x = torch.zeros((M, K), dtype=torch.bfloat16)
    out = torch.zeros((M, N), dtype=torch.bfloat16)
    total = sum(t.numel() * t.element_size() for t in (wq, s, b, x, out))
    assert bench.qmm_bytes(M, N, K, bits, gs) == total


def test_headline_bytes_and_measured_traffic():
    # Llama MLP shape, 4-bit g64, M = 1: 14336 x 4096 / 2 code bytes, one bf16
    # scale and bias per 64 weights, one bf16 x row, one bf16 out row.
    algo = bench.qmm_bytes(1, 14336, 4096, 4, 64)
    assert algo == 14336 * 2048 + 2 * 2 * 14336 * 64 + 2 * 4096 + 2 * 14336 == 33_067_008
    for t in (bench.MEASURED_TRAFFIC_QMM4_M1, bench.MEASURED_TRAFFIC_QMM4_M1_MLX):
        traffic = t["fetch_kib"] * 1024 * t["fetch_scale"] + t["write_kib"] * 1024 * t["write_scale"]
        # the kernel reads each weight byte once (repacked copy or MLX layout):
        # measured HBM traffic within 1% of it
        assert abs(traffic / algo - 1) < 0.01
