"""CPU restatement of the reference's prefill path: the parity oracle.

TEST INFRASTRUCTURE ONLY. Only tests/, `__graft_entry__.smoke()` and the
`cpu_baseline` leg of bench.py may import this package, and only as the
checker or the timed CPU baseline. The product (quail_amd) never imports
it and has no CPU fallback.

Modules:
  fp8.py        e4m3fn rounding and per-token group quantization
  qwen3_ref.py  the torch fp32 "dequantized path" of the Qwen3 forward pass
  packing_ref.py brute-force checks of pack layouts (prefix tree, pages, KV reads)
  pages_ref.py  the page accounting of the KV arena, in plain Python
  pack_ref.py   the unified pack layout, in plain Python
  labels_ref.py the label trie, its paths and each path row's context
"""
