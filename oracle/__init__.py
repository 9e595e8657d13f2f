"""CPU oracle for the fp8_flow_moe operator path -- TEST INFRASTRUCTURE ONLY.

Only ``tests/``, ``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of
``bench.py`` may import this package, and only as the checker or as the
reported CPU baseline.  The product (``nanopysche_amd``) never imports it and
has no CPU fallback: without the HIP library it raises.

Modules
-------
``oracle.fp8``      e4m3fn / e8m0 codecs and the blockwise quantisers
                    (1x128, 128x1, 128x128, MXFP8 1x32), dequantise and the
                    scaling-aware transpose -- numpy, bit-exact spec.
``oracle.routing``  softmax / sigmoid top-k gating, load-balancing loss,
                    stable counting sort, padded permute / unpermute.
``oracle.layer``    the expert block forward+backward: the BF16 per-expert
                    loop of the reference (fp32 torch CPU, autograd) and the
                    FP8 flow with the quantisation points the HIP path uses
                    (dequantise-then-fp32-matmul).

Pinning status of each function is recorded in each module's header.
"""
