"""sid on MI355X: the decode token loop of a small deterministic inference engine
(decode-verify-rollback), with every kernel on the path hand-written in HIP for gfx950.

Host API mirrors Aayaan-Sahu/deterministic-inference (`sid`): sid.config, sid.kernels.*,
sid.model.qwen3, sid.engine.*.
"""
