"""CPU oracle of the NCA hot path: test infrastructure, never the product.

Only `tests/`, `__graft_entry__.smoke()` and the `cpu_baseline` leg of `bench.py` may import
this package, and only to check or time against it. The product (`ncas_amd`) never imports it
and fails loudly when its HIP library is missing.

* `philox`      - Philox4x32-10 and the fire-mask rule in numpy (vectorised uint64 arithmetic);
* `clib`        - ctypes bindings of the C restatement (`nca_oracle.c`: Philox, the bit-exact
                  readout, conf@K selection), built by `oracle/Makefile`;
* `nca_oracle`  - the cell step and rollout restated in PyTorch-CPU from the reference's
                  `src/nca/model.py`, with injected fire masks and explicit bf16 rounding points.
"""
