"""The KLENT evaluator seams of the leaf-evaluation path (train.network_evaluate,
run.load_model); the self-play/fit orchestration around them is out of scope."""
