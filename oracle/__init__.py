"""CPU oracle for the batch-1 decode hot path.

TEST INFRASTRUCTURE ONLY.  Nothing in the product (``cudallm_amd``) imports, links or runs
anything from this package.  It may be used only by ``tests/``, by
``__graft_entry__.smoke()`` as the checker, and by ``bench.py``'s ``cpu_baseline`` leg.

Every function restates the reference's algorithm from its source (citations are
``path:line`` into the reference repository ``wasiqnauman/cudallm``):

* ``oracle.quantize``  - int8 per-row and int4 group-128 quantisers, pack/unpack, dequant
                         (``python/cudallm/quantize.py:5-47``).
* ``oracle.fileformat`` - the ``.cudallm`` reader/writer and tensor-name list
                         (``python/cudallm/format.py:7-147``, ``src/model/weights.cpp:66-81``).
* ``oracle.kernels``   - float64 closed forms of every single-kernel test hook
                         (``tests/test_kernels.py:19-207``; ``src/kernels/*.cu``).
* ``oracle.model``     - one decode step with an fp16 KV cache and greedy decoding
                         (``python/cudallm/reference.py:66-171``).
* ``oracle.synth``     - seeded synthetic model files (same tensors as
                         ``python/cudallm/export.py:85-159`` would write, from random bf16 masters).

How each part is pinned (checked against something other than itself):

* quantisers      - the reference's known-answer tests (``tests/test_quantize.py:10-63``) and
                    brute-force / invariant checks in ``tests/test_oracle.py``.
* file format     - struct sizes, byte-exact layout and name-list known answers
                    (``tests/test_format.py:31-106``) and the published ``weight_bytes`` known
                    answers (``results/decode/quant/Q_*.json``).
* kernel forms    - textbook identities (softmax sums to one, rotation preserves norms, the
                    single-token attention equals v, RMSNorm output has unit RMS ...).
* decode step     - golden vectors written by the reference's own ``ReferenceModel`` on tiny
                    seeded models (``tests/golden/make_decode_golden.py``), plus invariants.
"""
