"""Numeric constants of the per-layer quantization path.

Every value here is part of the output contract: the stored scales, the
zero-points and the integer codes depend on them bit for bit.  Values and
names follow ``converter/config.py:9-189`` of the reference so that code
written against the reference's constants keeps working.
"""

import torch

# Layer-name substrings that are stored unquantized (converter/config.py:11-18).
DEFAULT_SKIP_PATTERNS = [
    "embed",
    "norm",
    "modulation",
    "lm_head",
    "output",
    "proj_out",
]

# Symmetric scale divisors: largest positive code of each format.
INT4_SCALE_DIVISOR = 7.0
INT8_SCALE_DIVISOR = 127.0

# Stored scale dtype and its clamp range.  1e-5 is a subnormal in fp16 but
# survives the round trip with < 5 % error; 65500 stays below fp16 max.
SCALE_DTYPE = torch.float16
SMOOTH_FACTOR_DTYPE = torch.float16
SCALE_MIN = 1e-5
SCALE_MAX = 65500.0
FP16_SCALE_FLOOR = SCALE_MIN
MAX_FP16_SCALE = SCALE_MAX

# Floors used inside the LDLQ / GPTQ loops (never stored).
SCALE_FLOOR = 1e-8
DIAG_MEAN_FLOOR = 1e-6
DENOMINATOR_FLOOR = 1e-8
HINV_DIAG_FLOOR = 1e-8

# Normalised GPTQ error is clamped to +-100 (converter/rounding.py:91-92).
ERR_CLAMP_RANGE = 100.0

# Non-finite scale sanitisation in LDLQ.
SANITIZE_FLOOR = 1e-8
SANITIZE_CEIL = 1e30

# Weights with |w| above this are zeroed before rotation (converter/pipeline.py:527-537).
WEIGHT_OUTLIER_CLAMP = 1000.0

# LDLQ sign-flip threshold (a no-op for positive scales, kept for fidelity).
SIGN_FLIP_THRESHOLD = 1e-8

# Iterative LDLQ convergence control (converter/ldlq.py:479-550).
CONVERGENCE_EPS = 1e-10
CONVERGENCE_IMPROVEMENT_THRESHOLD = 1e-4
SCALE_FLOOR_MULTIPLIER = 0.1
SCALE_CEIL_MULTIPLIER = 10.0
ABS_SCALE_FLOOR = 1e-8
LDLQ_SCALE_MOMENTUM = 0.3
LDLQ_MSE_DIVERGENCE = 1.05
LDLQ_W_NONZERO = 1e-8

# Greedy search (converter/greedy.py, converter/config.py:128-151).
EIGENVALUE_FLOOR = 1e-12
STALL_THRESHOLD = 0.99
LOWRANK_MAX_RANK_FRAC = 0.3
LOWRANK_MAX_K = 512
INITIAL_BEST_COST = 1e30

SMOOTHQUANT_AMAX_FLOOR = 1e-8
SMOOTHQUANT_HESSIAN_FLOOR = SMOOTHQUANT_AMAX_FLOOR ** 2

# Column blocking of the full-rank greedy cross terms.
GREEDY_COL_BLOCK = 64
