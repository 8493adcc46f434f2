"""CPU oracle for the shifted-window Swin block forward of neural-scaling-weather.

TEST INFRASTRUCTURE ONLY.  Nothing in the product (the ``nsw`` package and the
HIP library ``libnsw.so``) imports, links or calls this package.  It is used
only by ``tests/``, ``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of
``bench.py``, always as the checker / CPU baseline and never as the thing that
is measured or shipped.

Modules
-------
``swin_ref``      fp32 PyTorch-on-CPU restatement of the reference block
                  (``models/swin_helpers.py``, ``models/mlp.py``,
                  ``models/layer_helpers.py``, ``distributed/mappings.py``,
                  ``distributed/helpers.py``), op for op, eager mode.
``index_maps``    numpy closed forms and brute-force loops for the integer
                  index work: cyclic roll, window partition / reverse, the
                  fused gather / scatter maps and the shift mask.
``metrics_ref``   numpy float64 latitude-weighted RMSE (``utils/losses.py``)
                  and the textbook latitude-weighted ACC, plus the cos-lat
                  area weights (``utils/misc_utils.py``).
``synth``         seeded synthetic inputs and reference-style weight init
                  (``models/timm_helpers.py`` trunc-normal).

How each function is pinned (beyond the restatement itself) is stated in the
module docstrings and checked by ``tests/test_oracle_*.py``.
"""
