"""scratchtape_amd: scratchtape's matrix-multiplication hot path on MI355X (gfx950).

Hand-written HIP kernels behind the C ABI of include/scratchtape_hip.h
(libscratchtape_hip.so, built in-tree by scratchtape_amd.build), with thin
Python mirrors of the reference interfaces they replace:

- matmul.MatRef / Epilogue / matmul / matmul_f32 / matmul_with  (gpu_step/matmul.rs)
- matmul.matmul_grouped: independent GEMMs in one launch          (gpu_step/tape.rs:324-347)
- tensor.ndarray_matmul                                         (src/tensor.rs NdArray::matmul)
- rows.softmax / softmax_backward / layer_norm(_backward)       (gpu_step/rows.rs)
- attention.step / fused_step (fused_forward, fused_backward)     (tape.rs:73-112, gpu_step/tape.rs)
- knn.KnnStore2bit (search_ivf, search_masked) / quantize_2bit / Centroids
                                                                (gpu_step/knn.rs, knn/ivf.rs)
- store.save / load: the 2-bit store in the reference's cache file format (gpu_step/knn/cache.rs)
"""
from ._lib import ScratchtapeError, lib  # noqa: F401
from .matmul import (Epilogue, MatRef, f16_enabled, f16_route, matmul, matmul_f32, matmul_grouped,  # noqa: F401
                     matmul_with, set_wait_limit, sync)

__all__ = ["ScratchtapeError", "lib", "MatRef", "Epilogue", "matmul", "matmul_f32", "matmul_with", "matmul_grouped",
           "f16_enabled", "f16_route", "sync", "set_wait_limit"]
