"""CPU oracle for the decode-phase quantized-KV path.

TEST INFRASTRUCTURE ONLY.  Nothing in the product imports this package: only
``tests/``, ``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of
``bench.py`` use it, and only as the checker / the timed CPU baseline.

It restates, on the CPU with PyTorch-CPU tensor ops (the reference path is
itself PyTorch), the arithmetic of zilangchen/LLM_KVCache_Quantization for:

* quantize-on-append (``quant.py``): INT8 symmetric static/dynamic, INT4
  symmetric static (+ adaptive / mixed / outlier-group rescue), nibble
  packing, and the asymmetric INT4 formula applied with static group
  parameters (the g32 + fp16-outlier-channel format, a build extension);
* decode attention (``attn.py``): the reference's torch decode oracle
  (fp16 dequant, fp32 einsum-softmax-einsum) and the dequant-then-attention
  oracle for the asymmetric g32 format.

Every function cites the reference ``file:line`` it follows.  How each one is
pinned (known-answer tests, closed forms, brute force, library routines) is
listed at the top of ``tests/test_oracle_pinning.py``.
"""
