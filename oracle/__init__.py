"""CPU oracle for the LoomFormer fused-kernel inference path.

TEST INFRASTRUCTURE ONLY.  Nothing in the product path (the HIP library, the
``kernels`` drop-in package, the ``loom_amd`` runtime) may import or call this
package.  Only ``tests/``, ``__graft_entry__.smoke()`` and the ``cpu_baseline``
leg of ``bench.py`` use it, and only as the checker (or the timed CPU
baseline), never as the thing that is measured or shipped.

The oracle is an fp32 PyTorch (CPU) restatement of the reference's *unfused*
PyTorch path: the functions each cite the reference ``file:line`` they follow
(paths relative to the reference checkout, srose69/Loomformer-Paraplex).

Pinning (what stops a plausible mistake in the restatement from passing):

* ``ops.py`` -- every op is checked in ``tests/test_oracle_golden.py`` against
  input/output vectors written by the reference itself (``tests/golden/``),
  and in ``tests/test_oracle_props.py`` against closed forms / invariants
  (tria.py self-test closed forms, RMS=1, PolARM fixed points, S=1 depth
  attention, compact-vs-dense W_imag brute force, endpoint == last row of the
  sequential carry, ...).
* ``model.py`` -- the seeded weight-init stream is pinned by per-tensor sha256
  of the reference's ``Model(cfg).state_dict()``; ``Model.step`` composition is
  pinned by the reference's own per-step logits and greedy ids on a tiny
  config (with the zero-initialised parameters perturbed so that inert paths
  are exercised) and by the greedy ids of the nano.yaml CPU-reference config.
"""
