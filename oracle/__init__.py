"""CPU oracle for causal / non-causal scaled-dot-product attention (fwd + bwd).

TEST INFRASTRUCTURE ONLY.  Nothing in the product path (``cudatransformer_amd``,
``include/``) imports, links or calls anything in this package.  Only ``tests/``,
``__graft_entry__.smoke()`` and ``bench.py``'s ``cpu_baseline`` leg use it, and only as
the checker (or the timed CPU comparator), never as the thing measured or shipped.

Contents
--------
``attention_fp64``  dense fp64 numpy restatement of the attention math that
                    ``flash_attention.cu`` (reference) computes, with the fixes the
                    reference lacks (causal flag, padded keys masked, correct dK/dV).
``c_oracle``        ctypes wrapper of ``attn_online.c``: a plain-C fp64 restatement of
                    the reference's *tiled online-softmax* loop structure
                    (``flash_attention.cu:97-161``) and of its recompute backward
                    (``flash_attention.cu:276-322``, with the dK/dV defect fixed).
``torch_cpu``       ``torch.nn.functional.scaled_dot_product_attention`` on CPU tensors:
                    the routine the reference's own test uses as its comparator
                    (``test_flash_attention.py:49``).  Used as a library cross-check in
                    fp64 and as the CPU baseline in fp32.

Pinning (what makes the oracle trustworthy) lives in ``tests/test_oracle.py``: the
two restatements against each other, against torch's SDPA autograd in fp64, against
closed forms / invariants, against central finite differences, and a planted-mistake
test showing that each check fails on a plausible bug.
"""
