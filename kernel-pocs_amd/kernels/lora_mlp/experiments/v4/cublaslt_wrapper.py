"""Import-path compatibility for callers of the reference's
kernels/lora_mlp/experiments/v4/cublaslt_wrapper.py: `cublaslt_matmul_epilogue`
keeps its name and signature, and runs on the MI355X epilogue GEMM
(`matmul_epilogue`, gemm_epilogue.py); no cuBLASLt is involved."""
from kernels.lora_mlp.experiments.v4.gemm_epilogue import matmul_epilogue as cublaslt_matmul_epilogue

__all__ = ["cublaslt_matmul_epilogue"]
