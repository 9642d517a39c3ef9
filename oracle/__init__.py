"""Parity oracle for femtochat's attention — TEST INFRASTRUCTURE ONLY.

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may
import this package, and only as the checker (or, for cpu_baseline, as the
reference CPU algorithm being timed).  The product path (femtochat_amd) never
imports or calls it, and it is never what a GPU measurement times.

* attention_ref.py : float64 dense restatement (mask, forward, backward).
* fa1.c / fa1.py   : float32 restatement of the reference's blocked
                     FlashAttention-1 CPU path (512 blocks, no skipping).
* rope_norm.py     : the attention prologue (rotary embedding, RMS norm x1.2).
* loss.py          : cross-entropy and its gradient, embedding gather and its
                     scatter-add gradient.

Every oracle function is pinned by tests/test_oracle.py against independent
library routines (torch autograd, scaled_dot_product_attention), finite
differences, closed forms and invariants; the reference itself ships no test
vectors (it has no tests).
"""
