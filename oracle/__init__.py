"""CPU oracle of the attention + norm hot path (test infrastructure only).

This package is the checker, never the product: only ``tests/``,
``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of ``bench.py`` may import it.
The product path (``kohakutt_amd``) never routes through it and fails loudly when its
HIP library is missing.

Everything here is float64 numpy, restating the reference's semantics:

* ``attention.sdpa`` -- dense SDPA with GQA/MQA head groups, top-left causal, bool and
  additive masks clamped at the reference's masked logit (-5e5), and the reference's
  fully-masked-row behaviour (softmax over the raw scores).
* ``attention.sdpa_varlen`` -- packed variable-length attention over ``cu_seqlens``
  with bottom-right causal alignment, the reference's offset validation, a ``[Tk]`` key
  mask and a per-sequence block-packed additive mask.
* ``norms.layer_norm`` / ``norms.rms_norm`` -- LayerNorm and RMSNorm over the last dim,
  with the statistics the reference's kernels return.
* ``ruler.diff_stats`` -- the float64 ruler: error statistics of a result against the
  float64 reference (the median relative error is what the parity bar bounds).

Pinning (which checks hold each function to something independent of this code) is
listed in each module's header.
"""

from . import attention, norms, ruler  # noqa: F401
