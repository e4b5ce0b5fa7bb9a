"""abacus.model_config: the reference's small default model dimensions (model_config.py)."""

DIM = 64
N_HEADS = 4
HEAD_DIM = 16
N_BLOCKS = 2
