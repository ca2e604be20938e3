"""CPU oracle for the MoE-layer hot path of SMEL FT — TEST INFRASTRUCTURE ONLY.

This package restates, on the CPU, what the reference computes on the path router -> dispatch -> int4/bf16+LoRA
expert GEMMs -> SiLU-gate -> combine (forward and backward). It is the checker for the HIP kernels and the timed CPU
baseline; it is never the product path. Only ``tests/``, ``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of
``bench.py`` may import it.

Modules
-------
``oracle.moe_ref``   torch (CPU) restatement in fp32 / fp64 of smel/moe.py, smel/lora.py and the int4 format of
                     smel/quant.py; autograd gives the backward, as in the reference's CPU path.
``oracle.norm_ref``  numpy fp32 restatement of the RMSNorm kernels of smel/norm.py (plain, residual add + norm,
                     gated; forward and backward) and of the torch code layer_runner.py runs instead of them.
``oracle.loss_ref``  the chunked cross-entropy's result from the full logits in fp64 (torch on the CPU).
``oracle.intref``    numpy restatement of the integer/byte parts (nibble unpacking, bf16 round-to-nearest-even,
                     stable counting-sort dispatch, lowest-index top-k) and a ctypes loader for the C restatement
                     ``oracle/c/oracle.c`` of the same functions.

Pinning (what checks each function against something other than itself): see the ``PINNED`` table in
``oracle.moe_ref``; every entry names the test that pins it. Functions marked "parity unpinned" there have no such
check.
"""
