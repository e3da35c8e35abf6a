"""Oracle for Aero's fused per-layer elementwise path.

TEST INFRASTRUCTURE ONLY. Only tests/, __graft_entry__.smoke() and bench.py's
cpu_baseline leg may import this package, and only to check the GPU results
(or as the timed CPU baseline). The product path in aero_amd/ never imports it.

`oracle.cpuref` binds the C restatement (cpuref.c, cpuref_quant.c).
`oracle.refbind` binds the reference's own C++ compiled into oracle/_ref/ by
`make -C oracle ref`, when that build exists; it cross-checks the oracle.
"""
