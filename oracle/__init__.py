"""CPU oracle for the FlashGRPO speculative rollout step.

THIS PACKAGE IS TEST INFRASTRUCTURE. It is a from-scratch numpy / Python
restatement of the reference algorithm (ihbkaiser/ss-GRPO, ``flashgrpo/``) and
exists only to check the HIP path. Only ``tests/``, ``__graft_entry__.smoke()``
and the ``cpu_baseline`` leg of ``bench.py`` may import it, and only as the
checker or as the timed CPU baseline. The product package (``flashgrpo_amd``)
never imports, calls or falls back to anything in here.

Modules and the reference code each follows:

* ``oracle.tree``      -- planner, dense candidate tree, tree-attention inputs
                          (``flashgrpo/decoding/medusa_tree.py:46-278``,
                          ``flashgrpo/decoding/tree_attention.py:6-67``,
                          ``flashgrpo/decoding/flash_medusa_decoder.py:341-412``)
* ``oracle.sampling``  -- supplied-noise sampler and the exact_target walk
                          (``flashgrpo/decoding/acceptance.py:7-260``,
                          ``flashgrpo_b200/decoding/acceptance.py:133-267``)
* ``oracle.kv``        -- accepted-path KV extraction
                          (``flashgrpo/decoding/kv_extraction.py:34-218``)
* ``oracle.model``     -- Medusa heads and the Qwen2/Llama tree-verify forward
                          (``flashgrpo/models/medusa_heads.py:12-87,241-290``,
                          ``flashgrpo/models/qwen_flashgrpo_wrapper.py:29-35,150-239``;
                          the decoder arithmetic itself lives in transformers 4.49)
* ``oracle.decode``    -- one verify step and the generate loop
                          (``flashgrpo/decoding/flash_medusa_decoder.py:550-1166``)

How each function is pinned (golden vectors, known answers, closed forms,
library cross-checks) is listed in ``tests/test_oracle_*.py``.
"""
