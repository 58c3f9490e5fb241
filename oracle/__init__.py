"""Test oracle for the paged-attention path. TEST INFRASTRUCTURE ONLY.

Nothing in `nimbus_amd/` imports this package. Only `tests/`,
`__graft_entry__.smoke()` and the `cpu_baseline` leg of `bench.py` may use it,
and only as the checker (or, for the CPU baseline, as the thing timed on the
host), never as a fallback for the HIP path.

Modules
-------
reference    CPU restatement of Nimbus's own PyTorch oracle
             (nimbus/kernels/reference.py:14-96): `index_copy_` slot write,
             block-table page gather, `scaled_dot_product_attention` with the
             reference's masks and `enable_gqa=True`. Also the per-row decode
             form used where the batched gather would not fit in host memory.
closed_form  float64 NumPy brute force of the same mathematics
             (softmax(q k^T * scale + mask) v, per sequence and head), written
             independently of torch's SDPA. It pins `reference`.

Parity status of each function (what pins it) is listed in each function's
docstring; every function here is pinned by a check in tests/test_oracle.py.
"""
