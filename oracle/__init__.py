"""CPU oracle for the fused LoRA linear path — TEST INFRASTRUCTURE ONLY.

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may import this
package, and only as the checker (or the timed CPU baseline), never as the code path
being measured or shipped. The product (weightshared_torchtitan_amd) never imports it.

Contents:
  lora_oracle   numpy float64 restatement of the reference LoRA-linear arithmetic,
                broadcast_add, fp8 e4m3fn quantisation, factorized embedding.
  qwen3_ref     torch-CPU float32 restatement of a weight-shared Qwen3 forward and of
                the reference's no-KV-cache greedy generation loop.

Pinning (what checks each function against something other than itself): see the
"Pinned by" line in each function's docstring. A function without one is marked
"parity unpinned" there.
"""
