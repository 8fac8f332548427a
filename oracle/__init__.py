"""CPU oracle for the paged-KV attention path.

TEST INFRASTRUCTURE ONLY. This package is a numpy restatement of MicroInfer's
own CPU/PyTorch reference path for paged attention, the KV append and the
block-table gather. It exists to check the HIP kernels, never to stand in for
them: only ``tests/``, ``__graft_entry__.smoke()`` and the ``cpu_baseline``
leg of ``bench.py`` may import it. The product package (``microinfer_amd``)
never imports it and has no CPU fallback.

Every function cites the reference file:line it follows and the checks that
pin it (see ``oracle/paged_attention.py`` module docstring).
"""

from oracle.numerics import (  # noqa: F401
    bf16_bits_to_f32,
    f32_to_bf16_bits,
    round_to_dtype,
)
from oracle.paged_attention import (  # noqa: F401
    dense_causal_attention_f64,
    gather_paged_kv,
    kv_append,
    merge_partials,
    paged_attention_reference,
    partial_attention_states,
    slot_indices,
)
