"""CPU oracle for the Boltz-2 Pairformer hot path.

TEST INFRASTRUCTURE ONLY.  Nothing in the product package (``tt-boltz_amd``)
imports this package.  It is imported by ``tests/``, by
``__graft_entry__.smoke()`` and by the ``cpu_baseline`` leg of ``bench.py``,
always as the checker (or as the timed CPU baseline), never as the thing that
is measured or shipped.

Contents
--------
``pairformer_ref``  fp32 PyTorch restatement of the reference CPU path
                    (``tt_bio/reference.py`` + primitives in ``tt_bio/boltz2.py``),
                    one function per reference module, each citing the lines it
                    follows.
``fp8_emu``         emulator of this build's ``--fast`` number format
                    (OCP e4m3 values, one power-of-two scale per 32 contiguous
                    elements along the contraction axis).  The reference has no
                    CPU fp8 path (``tt_bio/main.py:1648-1649``); this defines ours.
``msa_ref``         fp32 restatement of the MSA module (outer product mean, pair
                    weighted averaging, MSA layer, input embedding).
``diffusion_ref``   fp32 restatement of the pair side of the diffusion conditioning
                    (PairwiseConditioning, the token-transformer pair bias).
``brute``           scalar-loop restatements for tiny sizes (N <= 8), used by the
                    tests to pin ``pairformer_ref`` independently of torch's
                    einsum / matmul / softmax.

Parity pinning status (what checks each function, see ``tests/test_oracle.py``):
every function here is pinned by at least one of: brute-force loops at tiny N,
a library routine (``torch.nn.functional.scaled_dot_product_attention``,
``layer_norm``), or an invariant (transpose identities, masking, chunking
invariance, linearity, closed-form special cases).  No function is
"parity unpinned".
"""
