"""oracle -- CPU restatement of K100LC-RT4's quantized-matmul path.

TEST INFRASTRUCTURE ONLY.  Only tests/, __graft_entry__.smoke() and bench.py's
cpu_baseline leg may import anything from this package, and only as the checker
(or, in bench.py, as the timed CPU baseline); the product library never does.

  rt4_oracle.py   ctypes front end of liboracle.so (rt4_oracle.c, plain C)
  np_ref.py       independent numpy restatement + the numpy CPU baseline
  Makefile        builds liboracle.so and, where /root/reference exists, the
                  reference's own converter and kernels into _ref/
"""
