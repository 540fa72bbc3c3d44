"""CPU checks of bench.py's contract: one GPU only, the algorithmic-bytes rule that
`value` and `roofline.achieved` divide by, and the measured-traffic table."""
import os
import subprocess
import sys

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
sys.path.insert(0, ROOT)

import bench  # noqa: E402


def test_more_than_one_gpu_is_refused():
    p = subprocess.run([sys.executable, os.path.join(ROOT, "bench.py"), "--gpus", "2"],
                       stdout=subprocess.PIPE, stderr=subprocess.PIPE, text=True, timeout=300)
    assert p.returncode == 2
    assert "one GPU" in p.stderr
    assert p.stdout == ""


def test_algorithmic_bytes_per_launch():
    # weights once (34 bytes per 32-element block) + fp32 activations in + outputs out
    assert bench.gemv_bytes(8, 4096, 11008) == 4096 * 344 * 34 + 4 * 8 * 11008 + 4 * 8 * 4096
    assert bench.gemv_bytes(1, 12288, 4096) == 12288 * 128 * 34 + 4 * 4096 + 4 * 12288
    step = sum(bench.gemv_bytes(M, N, K) for M in bench.MS for _, N, K in bench.LLAMA_SET)
    assert step == 3 * sum(N * (K // 32) * 34 for _, N, K in bench.LLAMA_SET) + sum(
        4 * M * (K + N) for M in bench.MS for _, N, K in bench.LLAMA_SET)


def test_measured_traffic_table():
    for (layout, M, N, K), nbytes in bench.MEASURED_TRAFFIC.items():
        assert layout in ("raw", "tiled")
        # measured HBM bytes are at least the algorithmic bytes, and not wildly above;
        # the prefill GEMM reads W once per 256-row M tile (two tiles at M = 512)
        hi = 1.5 if M < 64 else 2.5
        assert 1.0 <= nbytes / bench.gemv_bytes(M, N, K) < hi, (layout, M, N, K)


def test_kernel_names_follow_the_path_choice():
    assert "gemv_rawk_kernel" in bench.decode_kernel_name(1, "raw", 4096, 11008)
    assert "gemv_q8_0_kernel" in bench.decode_kernel_name(1, "raw")
    assert "gemv_q8_0_kernel" in bench.decode_kernel_name(1, "raw", 151936, 896)
    assert "gemv_tiled_kernel" in bench.decode_kernel_name(1, "tiled", 4096, 11008)
    assert "gemv_tiled_kernel" in bench.decode_kernel_name(2, "tiled", 4096, 4096)
    assert "mfma" in bench.decode_kernel_name(2, "tiled", 151936, 896)
    assert "gemv_mfma_hyb_kernel" in bench.decode_kernel_name(8, "tiled", 4096, 11008)
    assert "gemv_mfma_hyb_kernel" in bench.decode_kernel_name(4, "tiled", 4096, 11008)
    assert "gemv_mfma_hyb_kernel" in bench.decode_kernel_name(8, "raw", 4096, 11008)
    assert "gemv_mfma_rows_kernel" in bench.decode_kernel_name(4, "raw", 12288, 4096)
    assert "gemv_q8_0_mfma_kernel" in bench.decode_kernel_name(8, "raw", 12288, 4096)
    assert "gemv_q8_0_mfma_kernel" in bench.decode_kernel_name(4, "raw", 4096, 4096)
    assert "gemv_q8_0_mfma_kernel" in bench.decode_kernel_name(8, "tiled", 4096, 4096)
    assert "gemv_mfma_rows_kernel" in bench.decode_kernel_name(8, "tiled", 12288, 4096)
    assert "gemv_mfma_rows_kernel" in bench.decode_kernel_name(4, "tiled", 11008, 4096)
    assert "gemv_q8_0_mfma_kernel" in bench.decode_kernel_name(5, "tiled", 11008, 4096)
    assert "gemv_q8_0_mfma_kernel" in bench.decode_kernel_name(8, "raw", 12288, 4096)
    assert "gemv_mfma_rows_kernel" in bench.decode_kernel_name(4, "tiled", 4096, 4096)
    assert "gemv_q8_0_mfma_kernel" in bench.decode_kernel_name(8, "tiled", 4096, 4096)
    assert "GEMM" in bench.decode_kernel_name(512, "tiled")
