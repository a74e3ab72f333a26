"""CPU oracle for the DeepSeek-Sparse-Attention hot path (TEST INFRASTRUCTURE ONLY).

This package restates, in numpy, the reference's host-side ground truth:

* ``lightning_indexer_ref``  <- lightning_indexer_numpy.py:20-111
  (plus the TND converters of lightning_indexer_triton.py:287-340)
* ``sparse_flash_attention_ref`` <- sparse_flash_attention_numpy.py:26-160
  (plus the TND / PA_BSND converters of sparse_flash_attention_triton.py:968-1051)
* ``sparse_flash_attention_grad_ref`` <- sparse_flash_attention_grad_numpy.py:34-143
  (plus the TND handling of sparse_flash_attention_grad_triton.py:562-674)

Only ``tests/``, ``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of
``bench.py`` may import it, and only as the checker / the timed CPU baseline.
The product path (``dsa_triton_ascend_amd``) never imports this package and
fails loudly when its HIP library is missing.

Pinning status (which independent checks fix each function) is listed in
``PINNING`` below and exercised by ``tests/test_oracle.py``.
"""

PINNING = {
    "numerics.round_bf16": "brute force vs torch fp32->bf16 (RNE) on special values and 2^20 random bit patterns",
    "numerics.quantize(fp16)": "numpy astype(float16) is IEEE RNE; checked against torch on random values",
    "lightning_indexer_ref.li_scores": "float64 einsum closed form on tiny shapes (GQA, odd N1, S1>S2)",
    "lightning_indexer_ref.li_golden_bsnd": "brute-force sorted((-score, idx)) tuples per row; mask closed forms "
                                            "(S1=1 sees key 0 only, rows >= act_q all -1, S1>S2 clamps at 0)",
    "lightning_indexer_ref.li_golden_tnd": "equivalence with per-batch BSND calls on the unpacked sequences",
    "sparse_flash_attention_ref.gather_positions": "hand-derived cases for bs=1/2/4, trailing -1 break, "
                                                   "scan limit ceil(threshold/bs), end>act_k clamp",
    "sparse_flash_attention_ref.sfa_golden_bsnd": "float64 torch.softmax attention on tiny shapes; "
                                                  "sm_max == max score, sm_sum >= 1; mode-3 leading rows zero",
    "sparse_flash_attention_ref.sfa_golden (TND/PA)": "equivalence with BSND after explicit de-packing / de-paging",
    "sparse_flash_attention_grad_ref.sfa_grad_golden_bsnd": "float64 torch autograd of the forward attention "
                                                            "(value a separate leaf) on tiny shapes, modes 0/3, "
                                                            "bs 1/2/4, actual lengths, a -1 inside a scan",
    "sparse_flash_attention_grad_ref.sparse_flash_attention_grad (TND)": "equivalence with per-batch BSND calls",
    "lightning_indexer_ref.lightning_indexer (PA_BSND)": "equivalence with BSND on the de-paged key cache",
    "sli_grad_kl_loss_ref.sli_grad_kl_loss": "float64 torch autograd of the KL loss on tiny shapes; the teacher "
                                             "built from exp(score - lse) over full keys; scipy rel_entr for the loss",
    "dense_loss_ref.dense_softmax_lse": "log(sum) + max equals scipy logsumexp over the visible keys; "
                                        "invisible rows keep (-inf, 0)",
    "dense_loss_ref.dense_loss_backward": "equals the sparse KL loss with every visible key as a slot (N2 = 1); "
                                          "with N2 = N1 the loss matches a per-head torch softmax teacher",
}
