"""Oracle: a CPU restatement of the reference's nnU-Net v2 inference path.

TEST INFRASTRUCTURE ONLY.  Only ``tests/``, ``__graft_entry__.smoke()`` and
``bench.py``'s ``cpu_baseline`` leg may import anything from this package, and only
as the checker (or as the timed CPU baseline), never as the product path.  The
product (``nnunet-mlx_amd/nnunet_mlx``) calls the HIP library and fails loudly when
it is missing; it never falls back to this code.

Modules:
  * ``network``        — torch-CPU float32 PlainConvUNet / ResidualEncoderUNet
                         following src/nnunet_mlx/model/network.py and
                         src/nnunet_mlx/kernels/metal_native_norm.py.
  * ``sliding_window`` — numpy restatement of src/nnunet_mlx/prediction/sliding_window.py
                         and the fold ensemble of src/nnunet_mlx/prediction/inference.py.
  * ``restore``        — numpy float64 restatement of the class-logit restoration
                         (half-pixel trilinear + argmax) of
                         src/nnunet_mlx/kernels/metal_restore.py.
  * ``preprocess``     — numpy restatement of raw-case preprocessing (crop to
                         nonzero, CT normalisation, the scikit-image / SciPy spline
                         resize and the separate-axis path) of
                         src/nnunet_mlx/data/preprocessing.py and resampling.py.

Pinning (what checks each function against something other than itself) is listed
in the module docstrings and exercised by ``tests/test_oracle_*.py``.  Nothing here
is "parity unpinned" except the bit-level agreement with MLX's own float32
summation orders, which no test in this environment can observe (MLX is absent).
"""
