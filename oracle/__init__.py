"""CPU oracle for the memory-layer lookup path.  TEST INFRASTRUCTURE ONLY.

This package restates, in numpy, the reference algorithm of the product-key
memory-layer lookup (KumarDev7/model ``memory_pool_model/memory.py``) and of
its sparse backward / row optimizer (``memory_pool_model/train.py``).  Every
function cites the reference file:line it follows.

It is a test oracle, never the product: only ``tests/``,
``__graft_entry__.smoke()`` and ``bench.py``'s ``cpu_baseline`` leg may import
it.  The product path (``model_amd``) never imports it and fails loudly when
its HIP library is missing.

How each function is pinned (the reference itself needs jax/flax/optax, which
are absent, so it cannot be executed):

* ``l2_normalize``            closed form in fp64 (tests/test_oracle.py)
* ``top_k``                   full stable argsort brute force + tie cases
* ``lookup_forward`` stage 1/2 brute force top-k over all n^2 slot sums
                              (the reference's own invariant, tests:40-52),
                              the flat-index tie rule on constructed ties
* softmax / gather / wsum     fp64 closed forms, sum(weights) == 1,
                              shuffle closed form (tests:577-588)
* ``aux_stats``               count sums (tests:30-37), balance-loss collapse
                              property (tests:153-160)
* ``lookup_backward``         torch-CPU autograd of an independent torch
                              restatement of the forward
* ``merge_rows`` etc.         scatter(sparse) == dense autograd gradient
                              (tests:321-344), unfetched rows exactly zero
* ``rowwise_adagrad``         known answer of tests:505-513
* ``lazy_adam``               closed-form first step (update == -lr*sign(g))
* ``warmup_cosine``           closed-form values at 0, warmup end, decay end
"""
