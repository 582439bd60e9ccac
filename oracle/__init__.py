"""CPU oracle of the routed-expert MoE layer.

TEST INFRASTRUCTURE ONLY: imported by tests/, __graft_entry__.smoke() and the
cpu_baseline leg of bench.py, always as the checker or the reported CPU
baseline, never by the product package (veystrix-core_amd/veymoe).

Modules:
  moe_oracle   NumPy restatement of the layer (float64 accumulation)
  ref_loops    pure-Python loop restatement of _numpy_projection (tiny shapes)
  pool_oracle  LRU slot table and record layout restatement
  cmoe.c       C restatement of the decode layer (OpenMP), the timed CPU baseline
"""
