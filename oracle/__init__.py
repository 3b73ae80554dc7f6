"""CPU oracle for the PPO update path — TEST INFRASTRUCTURE ONLY.

This package restates, on the CPU, the arithmetic of the reference's PPO
update (mrhooray/zero-to-hero, rl/deep/agents/ppo.py:113-193).  It exists to
check the MI355X library, never to stand in for it: only tests/,
__graft_entry__.smoke() and bench.py's cpu_baseline leg may import it, and
only as the checker or as the timed CPU baseline.  The product package
(ppo_amd) never imports it and fails loudly when its HIP library is missing.

Contents (each function cites the reference lines it follows):
  gae_ref.c            fp64 GAE recurrence, exact reference operation order
  ppo_oracle.py        Python/numpy/torch-CPU restatements of the whole path

How each piece is pinned (checked against something other than itself) is
stated in its docstring; tests/test_oracle.py carries those checks.
"""
