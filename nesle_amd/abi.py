"""ctypes binding of the C ABI in include/nesle_hip.h (libnesle_hip.so).

The lowest-level Python access to the HIP batch: plain pointers and sizes, no
pybind11.  The parity tests call the library through this module, and it is
the shape of binding a host program in another language would write against
the same header.  ``Batch`` raises ValueError / RuntimeError with the
library's message on failure, mirroring the reference binding's exceptions
(cpp/bindings/cuda_module.cu:185-189, 371-376).
"""

from __future__ import annotations

import ctypes
import re
from pathlib import Path

import numpy as np

PKG = Path(__file__).resolve().parent
LIB_PATH = PKG / "libnesle_hip.so"
INCLUDE = PKG.parent / "include"
HEADER = INCLUDE / "nesle_hip.h"

OK, EINVAL, ERUNTIME, EDEVICE = 0, 1, 2, 3
REWARD_SMB, REWARD_XDELTA = 0, 1
VIEW_RAM, VIEW_REWARDS, VIEW_DONES, VIEW_ACTIONS = 0, 1, 2, 3
VIEW_INSTRUCTIONS, VIEW_FRAMES, VIEW_BUDGET_HITS, VIEW_OPCODES, VIEW_PCS, VIEW_OAM = 4, 5, 6, 7, 8, 9
VIEW_FRAME_RGB, VIEW_FRAME_PALETTE, VIEW_GRAY84 = 10, 11, 12
VIEW_CENSUS = 13
VIEW_PRESENT = 14   # presentation records [n][16 + video memory block]
SHAPED_STATE_WORDS = 11   # NESLE_SMB_SHAPED_STATE_WORDS
# Step-kernel census slots (nesle_amd/csrc/nes_layout.h, namespace census).
CENSUS_FIELDS = ("waves", "iterations", "rare", "rare_io_write", "rare_side", "rare_idle", "rare_illegal",
                 "rare_timing", "rare_budget", "rare_outside", "rare_only_io_write", "dma", "present", "io_read",
                 "io_read_slow", "active_lanes", "distinct_entries", "cycles_loop", "cycles_rare", "cycles_io_read",
                 "lanes_io_write", "lanes_timing", "lanes_io_read", "lanes_io_read_slow", "exits",
                 "distinct_samples", "cycles_io_write", "cycles_settle", "cycles_dma", "cycles_present",
                 "cycles_redo", "redo")
FRAME_RGB, FRAME_PALETTE, FRAME_GRAY84 = 1, 2, 4
FRAME_LIVE = 8      # modifier: live state under the reference CPU core's rules
DTYPE_U8, DTYPE_I64, DTYPE_F32, DTYPE_U32, DTYPE_U64 = 0, 1, 2, 3, 4
STATE_BYTES = 22896
MAX_ENVS = 262144   # NESLE_MAX_ENVS

_U8P = ctypes.POINTER(ctypes.c_uint8)


class Config(ctypes.Structure):
    _fields_ = [
        ("num_envs", ctypes.c_uint32),
        ("frameskip", ctypes.c_uint32),
        ("max_instructions_per_frame", ctypes.c_uint32),
        ("reward_kind", ctypes.c_uint32),
        ("x_lo", ctypes.c_uint32),
        ("x_hi", ctypes.c_uint32),
        ("done_addr", ctypes.c_uint32),
        ("clip", ctypes.c_uint32),
        ("time_penalty", ctypes.c_float),
        ("device", ctypes.c_int32),
        ("frames", ctypes.c_uint32),
    ]


class View(ctypes.Structure):
    _fields_ = [
        ("data", ctypes.c_void_p),
        ("ndim", ctypes.c_int32),
        ("shape", ctypes.c_int64 * 4),
        ("dtype", ctypes.c_int32),
        ("device_id", ctypes.c_int32),
    ]


class ShapedParams(ctypes.Structure):
    """nesle_smb_shaped_params (include/nesle_ppo.h)."""
    FLOATS = ("progress_scale", "backtrack_scale", "checkpoint_bonus", "checkpoint_width", "score_scale",
              "coin_bonus", "kill_bonus", "finish_zone_x", "finish_zone_bonus", "flag_zone_x", "flag_bonus",
              "death_penalty", "time_penalty", "stall_penalty", "max_stall_penalty", "jump_penalty",
              "neutral_jump_penalty", "repeated_jump_penalty", "max_repeated_jump_penalty", "left_penalty",
              "bad_button_penalty")
    _fields_ = [(name, ctypes.c_float) for name in FLOATS] + [("stall_window", ctypes.c_int32),
                                                              ("repeated_jump_window", ctypes.c_int32)]


class RomInfo(ctypes.Structure):
    _fields_ = [(name, ctypes.c_uint32) for name in (
        "prg_rom_size", "chr_rom_size", "mapper", "submapper", "nametable_arrangement",
        "has_trainer", "has_battery", "is_nes2")]


_LIB = None


def bind_runtime() -> None:
    """Load PyTorch (when installed) before libnesle_hip.so.

    PyTorch-ROCm ships its own libamdhip64.so (SONAME libamdhip64.so.7).  If
    it is already loaded, libnesle_hip.so's dependency on that SONAME binds to
    it and the process has one HIP runtime, so device pointers pass freely
    between torch and the batch.  Loaded the other way round, two runtimes
    would compete for the GPU.
    """
    try:
        import torch  # noqa: F401
    except ImportError:
        pass


def declared_functions() -> list[str]:
    """Names of every function the headers under include/ declare."""
    names: set[str] = set()
    for header in sorted(INCLUDE.glob("*.h")):
        text = re.sub(r"/\*.*?\*/", "", header.read_text(), flags=re.S)
        names.update(re.findall(r"\b(nesle_[a-z0-9_]+)\s*\(", text))
    return sorted(names)


def lib():
    """Load libnesle_hip.so (fails loudly when it has not been built)."""
    global _LIB
    if _LIB is not None:
        return _LIB
    if not LIB_PATH.exists():
        raise ImportError(f"{LIB_PATH} is missing: run `python -m nesle_amd.build`")
    bind_runtime()
    L = ctypes.CDLL(str(LIB_PATH))
    vp = ctypes.c_void_p
    sig = {
        "nesle_config_init": (None, [ctypes.POINTER(Config)]),
        "nesle_create": (ctypes.c_int, [ctypes.POINTER(Config), ctypes.c_char_p, ctypes.c_size_t, ctypes.POINTER(vp)]),
        "nesle_create_synthetic": (ctypes.c_int, [ctypes.POINTER(Config), ctypes.POINTER(vp)]),
        "nesle_synthetic_step": (ctypes.c_int, [vp, ctypes.c_int, ctypes.c_int]),
        "nesle_set_snapshots": (ctypes.c_int, [vp, ctypes.POINTER(ctypes.c_char_p), ctypes.POINTER(ctypes.c_size_t),
                                               ctypes.c_uint32, _U8P]),
        "nesle_retain": (None, [vp]),
        "nesle_release": (None, [vp]),
        "nesle_reset": (ctypes.c_int, [vp]),
        "nesle_reset_envs": (ctypes.c_int, [vp, vp, ctypes.c_int]),
        "nesle_set_actions": (ctypes.c_int, [vp, vp, ctypes.c_int, ctypes.c_int]),
        "nesle_step": (ctypes.c_int, [vp, ctypes.c_int, ctypes.c_int]),
        "nesle_get_view": (ctypes.c_int, [vp, ctypes.c_int, ctypes.POINTER(View)]),
        "nesle_copy_to_host": (ctypes.c_int, [vp, ctypes.c_int, vp, ctypes.c_size_t]),
        "nesle_render": (ctypes.c_int, [vp, ctypes.c_uint32]),
        "nesle_save_state": (ctypes.c_int, [vp, ctypes.c_uint32, _U8P]),
        "nesle_load_state": (ctypes.c_int, [vp, ctypes.c_char_p, ctypes.c_size_t, _U8P]),
        "nesle_snapshot_capture": (ctypes.c_int, [vp, ctypes.c_uint32, ctypes.c_uint32]),
        "nesle_snapshot_export": (ctypes.c_int, [vp, ctypes.c_uint32, _U8P]),
        "nesle_set_env_levels": (ctypes.c_int, [vp, _U8P]),
        "nesle_poke_ram": (ctypes.c_int, [vp, ctypes.c_uint32, ctypes.c_uint32]),
        "nesle_poke_ram_envs": (ctypes.c_int, [vp, ctypes.c_uint32, vp, ctypes.c_int]),
        "nesle_synchronize": (ctypes.c_int, [vp]),
        "nesle_set_stream": (ctypes.c_int, [vp, vp]),
        "nesle_num_envs": (ctypes.c_uint32, [vp]),
        "nesle_frameskip": (ctypes.c_uint32, [vp]),
        "nesle_num_levels": (ctypes.c_uint32, [vp]),
        "nesle_device_id": (ctypes.c_int32, [vp]),
        "nesle_set_timing": (ctypes.c_int, [vp, ctypes.c_int]),
        "nesle_get_timing": (ctypes.c_int, [vp, ctypes.POINTER(ctypes.c_double), ctypes.POINTER(ctypes.c_uint64)]),
        "nesle_get_timing_split": (ctypes.c_int, [vp, ctypes.POINTER(ctypes.c_double), ctypes.POINTER(ctypes.c_double),
                                                  ctypes.POINTER(ctypes.c_uint64)]),
        "nesle_parse_ines": (ctypes.c_int, [ctypes.c_char_p, ctypes.c_size_t, ctypes.POINTER(RomInfo)]),
        "nesle_parse_fcs": (ctypes.c_int, [ctypes.c_char_p, ctypes.c_size_t, _U8P]),
        "nesle_last_error": (ctypes.c_char_p, []),
        "nesle_ppo_head_scratch_floats": (ctypes.c_uint32, [ctypes.c_uint32]),
        "nesle_ppo_head": (ctypes.c_int, [vp, vp, vp, vp, vp, vp, ctypes.c_uint32, ctypes.c_uint32, ctypes.c_double,
                                          ctypes.c_double, ctypes.c_double, vp, vp, vp, vp, vp, vp, vp]),
        "nesle_ppo_head_static": (ctypes.c_int, [vp, vp, vp, vp, vp, vp, ctypes.c_uint32, ctypes.c_uint32,
                                                 ctypes.c_double, ctypes.c_double, ctypes.c_double, vp, vp, vp, vp,
                                                 vp, vp]),
        "nesle_smb_shaped_defaults": (None, [ctypes.POINTER(ShapedParams)]),
        "nesle_smb_shaped_reset": (ctypes.c_int, [vp, vp, ctypes.c_uint32, vp, vp]),
        "nesle_smb_shaped_reward": (ctypes.c_int, [vp, vp, vp, ctypes.c_uint32, ctypes.POINTER(ShapedParams), vp,
                                                   vp, vp]),
    }
    for name, (res, args) in sig.items():
        fn = getattr(L, name)
        fn.restype = res
        fn.argtypes = args
    _LIB = L
    return L


def _check(rc: int) -> None:
    if rc == OK:
        return
    msg = lib().nesle_last_error().decode()
    if rc == EINVAL:
        raise ValueError(msg)
    raise RuntimeError(msg)


def parse_ines(rom: bytes) -> dict:
    info = RomInfo()
    _check(lib().nesle_parse_ines(rom, len(rom), ctypes.byref(info)))
    return {name: getattr(info, name) for name, _ in RomInfo._fields_}


def parse_fcs(data: bytes) -> np.ndarray:
    out = np.zeros(STATE_BYTES, dtype=np.uint8)
    _check(lib().nesle_parse_fcs(data, len(data), out.ctypes.data_as(_U8P)))
    return out


class Batch:
    """Owning handle over one ``nesle_batch``."""

    def __init__(self, rom: bytes | None, num_envs: int, frameskip: int = 4, *, reward_kind: int = REWARD_SMB,
                 x_lo: int = 0x86, x_hi: int = 0x6D, done_addr: int = 0, clip: int = 15,
                 time_penalty: float = 0.0, max_instructions_per_frame: int = 0, device: int = -1,
                 frames: bool = True) -> None:
        """``rom`` None: the ROM-less synthetic batch (nesle_create_synthetic)."""
        L = lib()
        cfg = Config()
        L.nesle_config_init(ctypes.byref(cfg))
        cfg.num_envs, cfg.frameskip = num_envs, frameskip
        cfg.max_instructions_per_frame = max_instructions_per_frame
        cfg.reward_kind, cfg.x_lo, cfg.x_hi, cfg.done_addr, cfg.clip = reward_kind, x_lo, x_hi, done_addr, clip
        cfg.time_penalty = time_penalty
        cfg.device = device
        cfg.frames = int(frames)
        h = ctypes.c_void_p()
        if rom is None:
            _check(L.nesle_create_synthetic(ctypes.byref(cfg), ctypes.byref(h)))
        else:
            _check(L.nesle_create(ctypes.byref(cfg), rom, len(rom), ctypes.byref(h)))
        self.h = h
        self.n = num_envs

    def close(self) -> None:
        if getattr(self, "h", None):
            lib().nesle_release(self.h)
            self.h = None

    def __del__(self) -> None:
        self.close()

    def set_snapshots(self, blobs: list[bytes], env_to_level: np.ndarray | None = None) -> None:
        arr = (ctypes.c_char_p * len(blobs))(*blobs)
        lens = (ctypes.c_size_t * len(blobs))(*[len(b) for b in blobs])
        lv = None
        if env_to_level is not None:
            lv = np.ascontiguousarray(env_to_level, dtype=np.uint8)
            lv_ptr = lv.ctypes.data_as(_U8P)
        else:
            lv_ptr = None
        _check(lib().nesle_set_snapshots(self.h, arr, lens, len(blobs), lv_ptr))
        del lv

    def set_actions(self, actions) -> None:
        """Host numpy uint8/int64 array, or a device tensor (torch)."""
        if isinstance(actions, np.ndarray):
            a = np.ascontiguousarray(actions)
            dtype = DTYPE_I64 if a.dtype == np.int64 else DTYPE_U8
            if dtype == DTYPE_U8:
                a = a.astype(np.uint8, copy=False)
            assert a.shape == (self.n,)
            _check(lib().nesle_set_actions(self.h, a.ctypes.data, dtype, 0))
        else:
            dtype = DTYPE_I64 if str(actions.dtype) == "torch.int64" else DTYPE_U8
            _check(lib().nesle_set_actions(self.h, actions.data_ptr(), dtype, 1))

    def step(self, auto_reset: bool = False, stats_mode: int = 0) -> None:
        _check(lib().nesle_step(self.h, int(auto_reset), stats_mode))

    def synthetic_step(self, apply_actions: bool = True, auto_reset: bool = False) -> None:
        _check(lib().nesle_synthetic_step(self.h, int(apply_actions), int(auto_reset)))

    def census(self) -> dict:
        """The step kernel's census of the last stats-mode-3 step, by name."""
        raw = self.host(VIEW_CENSUS)
        return {name: int(raw[i]) for i, name in enumerate(CENSUS_FIELDS)}

    def reset(self) -> None:
        _check(lib().nesle_reset(self.h))

    def reset_envs(self, mask: np.ndarray) -> None:
        m = np.ascontiguousarray(mask, dtype=np.uint8)
        _check(lib().nesle_reset_envs(self.h, m.ctypes.data, 0))

    def view(self, kind: int) -> View:
        v = View()
        _check(lib().nesle_get_view(self.h, kind, ctypes.byref(v)))
        return v

    def host(self, kind: int) -> np.ndarray:
        if kind == VIEW_PRESENT:
            v = self.view(kind)
            out = np.empty((self.n, int(v.shape[1])), dtype=np.uint8)
            _check(lib().nesle_copy_to_host(self.h, kind, out.ctypes.data, out.nbytes))
            return out
        dt = {VIEW_RAM: (np.uint8, (self.n, 2048)), VIEW_REWARDS: (np.float32, (self.n,)),
              VIEW_DONES: (np.uint8, (self.n,)), VIEW_ACTIONS: (np.uint8, (self.n,)),
              VIEW_INSTRUCTIONS: (np.uint64, (self.n,)), VIEW_FRAMES: (np.uint32, (self.n,)),
              VIEW_BUDGET_HITS: (np.uint32, (self.n,)), VIEW_OPCODES: (np.uint64, (256,)),
              VIEW_PCS: (np.uint64, (65536,)), VIEW_OAM: (np.uint8, (self.n, 256)),
              VIEW_FRAME_RGB: (np.uint8, (self.n, 240, 256, 3)), VIEW_FRAME_PALETTE: (np.uint8, (self.n, 240, 256)),
              VIEW_GRAY84: (np.uint8, (self.n, 84, 84)), VIEW_CENSUS: (np.uint64, (32,))}[kind]
        out = np.empty(dt[1], dtype=dt[0])
        _check(lib().nesle_copy_to_host(self.h, kind, out.ctypes.data, out.nbytes))
        return out

    def render(self, outputs: int = FRAME_RGB) -> None:
        """Draw every console's presentation snapshot into the FRAME_* outputs."""
        _check(lib().nesle_render(self.h, outputs))

    def save_state(self, env: int) -> np.ndarray:
        out = np.empty(STATE_BYTES, dtype=np.uint8)
        _check(lib().nesle_save_state(self.h, env, out.ctypes.data_as(_U8P)))
        return out

    def load_state(self, state, mask: np.ndarray | None = None) -> None:
        raw = bytes(np.asarray(state, dtype=np.uint8)) if not isinstance(state, bytes) else state
        m = None if mask is None else np.ascontiguousarray(mask, dtype=np.uint8)
        _check(lib().nesle_load_state(self.h, raw, len(raw), None if m is None else m.ctypes.data_as(_U8P)))

    def snapshot_capture(self, env: int, slot: int) -> None:
        _check(lib().nesle_snapshot_capture(self.h, env, slot))

    def snapshot_export(self, slot: int) -> np.ndarray:
        out = np.empty(STATE_BYTES, dtype=np.uint8)
        _check(lib().nesle_snapshot_export(self.h, slot, out.ctypes.data_as(_U8P)))
        return out

    def set_env_levels(self, levels: np.ndarray) -> None:
        lv = np.ascontiguousarray(levels, dtype=np.uint8)
        _check(lib().nesle_set_env_levels(self.h, lv.ctypes.data_as(_U8P)))

    def poke_ram(self, address: int, value: int) -> None:
        _check(lib().nesle_poke_ram(self.h, address, value))

    def poke_ram_envs(self, address: int, values: np.ndarray) -> None:
        """RAM[address] of console e = values[e] (host uint8, one per console)."""
        v = np.ascontiguousarray(values, dtype=np.uint8)
        assert v.shape == (self.n,)
        _check(lib().nesle_poke_ram_envs(self.h, address, v.ctypes.data, 0))

    def synchronize(self) -> None:
        _check(lib().nesle_synchronize(self.h))

    def set_stream(self, stream_ptr: int) -> None:
        _check(lib().nesle_set_stream(self.h, stream_ptr))

    def set_timing(self, enable: bool) -> None:
        _check(lib().nesle_set_timing(self.h, int(enable)))

    def timing(self) -> tuple[float, int]:
        """(summed step-kernel milliseconds, timed launches) since enabling."""
        ms = ctypes.c_double()
        n = ctypes.c_uint64()
        _check(lib().nesle_get_timing(self.h, ctypes.byref(ms), ctypes.byref(n)))
        return ms.value, n.value

    def timing_split(self) -> tuple[float, float, int]:
        """(step-kernel ms, auto-reset restore-kernel ms, timed steps) since enabling."""
        ms, reset_ms, n = ctypes.c_double(), ctypes.c_double(), ctypes.c_uint64()
        _check(lib().nesle_get_timing_split(self.h, ctypes.byref(ms), ctypes.byref(reset_ms), ctypes.byref(n)))
        return ms.value, reset_ms.value, n.value

    @property
    def num_levels(self) -> int:
        return lib().nesle_num_levels(self.h)
