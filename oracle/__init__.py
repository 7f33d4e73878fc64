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
      tests/golden/known_answers.json (executor strided pack
      [0,1,2,6,7,8,3,4,5,9,10,11], scratch tail, replicated x0.5) and the
      invariant sum(exact_numel) == sum(numel)   [test_grad_sync_host.py]
  gradsync.l2_norm / clip / inf_norm / count_zeros
                                   -> [3,4,0,0] -> 5.0 -> [1.2,1.6,0,0],
      zeros 2, inf-norm 1.6 (golden)
  gradsync.unscale_and_check       -> non-finite flag and the exact
      power-of-two scale (closed forms)
  adamw.adamw_step                 -> torch.optim.AdamW (third-party, the
      reference's FusedAdam fallback) and the step-1 closed form
      m = 0.1 g, v = 0.05 g^2 (golden)
  adamw.to_bf16                    -> torch's round-to-nearest-even cast
  layer.layer_norm / bias_gelu     -> eps 1e-5 and tanh-GELU closed values
  layer.causal_attention           -> the explicit masked softmax (fp64)
  layer.vocab_cross_entropy        -> F.cross_entropy at the reference's own
      bar (13x17 rows, V 11, logits x1000, error < 1e-6; the unshifted
      form fails it) and ln V for uniform logits
  layer.transformer_layer          -> closed forms: zero weights give
      x + proj_b + fc2_b; per-head q|k|v split; causal running mean along
      the sequence axis; MLP = fc2 gelu(fc1 bias); gradients by gradcheck
  layer.middle_stage_fwd_bwd       -> central differences of <stage(x), dy>
  layer.full_model_fwd_bwd         -> zero tied head: loss ln V and the
      closed-form tied gradient; central differences along the word table
      (tied sum), position table, final LN and a layer weight
  [test_oracle_pins.py, test_grad_sync_host.py]
"""
