"""CPU oracle of the Motif decode-attention hot path — test infrastructure only.

``oracle.oracle`` is the numpy restatement used as the checker; ``oracle.c_oracle``
binds the C/OpenMP restatement (``motif_oracle.c``) used as a second check and
as the timed CPU baseline.  Only tests/, __graft_entry__.smoke() and bench.py's
cpu_baseline leg may import this package; the product never does.
"""
