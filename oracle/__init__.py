"""CPU parity oracle for the testt_amd kernel set -- TEST INFRASTRUCTURE ONLY.

A restatement, on the CPU, of the reference's algorithm for each kernel of the QLoRA fused
set of SalReII/testt `solution/`, in the reference's own operation order, and of the eager
PyTorch path those kernels replace (bitsandbytes dequant, transformers' Qwen2RMSNorm and
apply_rotary_pos_emb, SiLU * up, cross-entropy):

- nf4.py      NF4 double-quant dequant (numpy fp32, each product/sum rounded) + a bitsandbytes-
              style quantizer that builds realistic quant states for the tests
- rmsnorm.py  residual add + Qwen2RMSNorm forward, backward by torch autograd (CPU)
- rope.py     LoRA add + index_copy into the padded layout + apply_rotary_pos_emb, backward by
              autograd (CPU)
- swiglu.py   F.silu(g) * u forward, backward by autograd (CPU)
- head.py     log-softmax statistics, argmax and (softmax - onehot) * scale in float64

Only tests/, __graft_entry__.smoke() and bench.py's CPU-baseline leg may import this package,
and only as the checker or the timed CPU baseline; the product path (testt_amd) never does.

Pinning (how each function is checked independently of its own formula): see the module
docstrings and tests/test_oracle_*.py.  Every function here is pinned; none is "parity
unpinned" except where a module docstring says so.
"""
