"""CPU oracle of the ReplaySSM GDN decode path -- TEST INFRASTRUCTURE ONLY.

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may import
this package; the product (fp8-replayssm-gdn-kernel_amd/) never does.

  gdn_oracle   numpy restatement of the reference algorithm (file:line cited
               per function)
  fp8_quant    ctypes bindings of fp8_quant.c, an independent integer-arithmetic
               restatement of the vblock32 quantiser
"""
