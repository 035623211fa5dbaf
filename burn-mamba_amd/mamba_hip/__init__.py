"""mamba_hip — host side of the MI355X (gfx950) SSM hot path for burn-mamba.

Thin Python mirror of the reference's operator interfaces over the C ABI of
libmamba_hip.so (include/mamba_hip.h).  Every compute call goes to the HIP
library; nothing here computes on the CPU.
"""

from ._lib import MambaHipError, exported_symbols, lib  # noqa: F401
from .mamba1 import (Mamba1, Mamba1Cache, Mamba1Config, conv1d_fwd, conv1d_step, mamba1_scan, scan_step,  # noqa: F401
                     selective_scan, selective_scan_step)
from .ssd import Mamba2SsdInput, Mamba2SsdPath, ssd2_fast_path, ssd2_fwd  # noqa: F401
from .ssd import ssd2_autograd, ssd2_bwd  # noqa: F401
from .step import (Mamba2, Mamba2Cache, Mamba2Config, Mamba2Layer, Mamba2Stack, linear, pack_linear,  # noqa: F401
                   rmsnorm, step_ssm, step_ssm_args)
from .step import conv_fwd as mamba2_conv_fwd, div_eps, gated_rmsnorm as mamba2_gated_rmsnorm  # noqa: F401
from .step import batch_parts, drop_derived, packed_weight, prefill_mm, step_mm, step_mm_ok  # noqa: F401
from .ssd3 import (Mamba3DoubleSsdInput, Mamba3SingleSsdInput, ssd3_double_fast_path, ssd3_double_fwd,  # noqa: F401
                   ssd3_autograd, ssd3_bwd, ssd3_fast_path, ssd3_fwd)
from .mamba3 import Mamba3, Mamba3Cache, Mamba3Config, Mamba3Layer, Mamba3Stack  # noqa: F401
from .mamba3 import step_ssm as mamba3_step_ssm, step_ssm_args as mamba3_step_ssm_args  # noqa: F401
from .mamba3 import finish_fwd as mamba3_finish_fwd, prep_fwd as mamba3_prep_fwd  # noqa: F401
from .mamba3 import prep_args as mamba3_prep_args, prep_fast_path as mamba3_prep_fast_path  # noqa: F401
from .mamba3 import double_inputs as mamba3_double_inputs  # noqa: F401
from .mamba3 import fused_args as mamba3_fused_args, fused_supported as mamba3_fused_supported  # noqa: F401
from .mamba3 import fused_run as mamba3_fused_run, ssd_fused_fwd as mamba3_ssd_fused_fwd  # noqa: F401
