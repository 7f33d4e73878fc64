"""CPU oracle for the eth_amd hot path -- TEST INFRASTRUCTURE ONLY.

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may
import anything under oracle/, and only as the checker (or the timed CPU
baseline), never as the product path.  The product (eth_amd) has no CPU
fallback and never imports this package.

Modules:
  gradsync  -- numpy restatement of bucket pack / all-reduce seam / normalize /
               unpack, unscale + inf/nan flag, canonical L2 norm + clip
  adamw     -- numpy restatement of torch.optim.AdamW (decoupled weight decay)
  layer     -- torch-CPU (fp32/fp64) restatement of the GPT layer ops and of
               one middle-stage forward/backward

Pinning (what each function is checked against, in tests/):
  gradsync.pack_bucket / execute   -> reference known answers restated in
      tests/golden/grad_sync_known_answers.json (executor strided pack
      [0,1,2,6,7,8,3,4,5,9,10,11], scratch tail, replicated x0.5) and the
      invariant sum(exact_numel) == sum(numel)
  gradsync.l2_norm / clip          -> [3,4,0,0] -> 5.0 -> [1.2,1.6,0,0],
      zeros 2, inf-norm 1.6 (golden); fp64 brute force
  adamw.adamw_step                 -> torch.optim.AdamW (third-party, the
      reference's FusedAdam fallback) and the step-1 closed form
      m = 0.1 g, v = 0.05 g^2 (golden)
  layer.*                          -> torch.nn.functional (F.layer_norm,
      F.gelu(tanh), F.scaled_dot_product_attention(is_causal),
      F.cross_entropy) and fp64 brute force on tiny shapes
"""
