"""RL / infinite-context operators (mirroring ``flashrwkv2.rl_infctx``)."""
