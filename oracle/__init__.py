"""CPU oracle for the CacheBridge online handoff path (map + paged install).

TEST INFRASTRUCTURE ONLY. This package is a CPU restatement of the reference
algorithm, used as the checker for the HIP implementation in
``cachebridge_amd``. Only ``tests/``, ``__graft_entry__.smoke()`` and the
``cpu_baseline`` leg of ``bench.py`` may import it, and only to check or to
time the reference algorithm on the CPU. The product path never imports,
calls or falls back to anything here.

Modules and the reference code each one restates (paths relative to the
reference repository root; ``cb/`` = ``src/cachebridge/``):

- ``oracle.rope``    -- ``cb/rope.py:9-89`` (split-half RoPE, YaRN tables,
  rotate / un-rotate), op for op in torch fp32.
- ``oracle.mapper``  -- ``cb/mapper.py:17-239`` (``PageMapper``: artifact load,
  TP head slice, ``map_page``) and the head-local view
  ``cb/online/mapping.py:6-33``.
- ``oracle.install`` -- ``cb/online/blocks.py:47-111`` (``pack_source_block``,
  ``map_write_block``), a row-store restatement of SGLang's
  ``MHATokenToKVPool.set_kv_buffer`` (SGLang v0.4.10.post2, un-vendored),
  the virtual-page construction for per-(layer, head) source assignments,
  and ``cb/architectures/gemma3.py:39-58`` window materialisation.
- ``oracle.structured`` -- ``cb/architectures/qwen35.py:52-61``
  (``transform_delta_state``), in float64 numpy.

Parity status of each function is stated in its docstring; "parity pinned"
names the golden vectors or closed forms that check it in ``tests/``.
"""
