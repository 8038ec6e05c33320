"""The C ABI of libnesle_hip.so without a GPU: the library loads, exports every
function the headers under include/ declare, and its host-only entry points
(iNES/FCS parsing, argument validation) behave like the reference binding's
(cpp/src/rom.cpp:65-121, cpp/bindings/cuda_module.cu:371-376)."""

from __future__ import annotations

import ctypes

import pytest

from nesle_amd import abi, synthrom


def _ines(trainer=False, prg_banks=2, chr_banks=1, flags6=0, flags7=0, flags8=0, flags9=0) -> bytes:
    """The image tests/cpp/test_core.cpp:11-29 builds."""
    h = bytearray(b"NES\x1a") + bytes([prg_banks, chr_banks, flags6 | (0x04 if trainer else 0), flags7,
                                       flags8, flags9]) + bytes(6)
    body = (b"T" * 512 if trainer else b"") + b"P" * (prg_banks * 16384) + b"C" * (chr_banks * 8192)
    return bytes(h) + body


def test_library_exports_every_declared_function():
    lib = abi.lib()
    names = abi.declared_functions()
    assert len(names) >= 25
    missing = [n for n in names if not hasattr(lib, n)]
    assert not missing, f"declared but not exported: {missing}"


def test_binding_constants_match_the_header():
    text = abi.HEADER.read_text()
    assert f"#define NESLE_MAX_ENVS {abi.MAX_ENVS}u" in text


def test_parse_ines_known_answers():
    """tests/cpp/test_core.cpp:33-100."""
    info = abi.parse_ines(_ines())
    assert (info["mapper"], info["submapper"], info["prg_rom_size"], info["chr_rom_size"]) == (0, 0, 32768, 8192)
    assert abi.parse_ines(_ines(trainer=True))["has_trainer"] == 1
    assert abi.parse_ines(_ines(flags6=0x10))["mapper"] == 1
    nes2 = abi.parse_ines(_ines(flags7=0x08))
    assert nes2["is_nes2"] == 1 and nes2["mapper"] == 0
    assert abi.parse_ines(_ines(flags7=0x08, flags8=0x10))["submapper"] == 1
    with pytest.raises(ValueError, match="extended"):
        abi.parse_ines(_ines(flags7=0x08, flags9=0x01))
    with pytest.raises(ValueError, match="shorter"):
        abi.parse_ines(b"NES\x1a")
    with pytest.raises(ValueError, match="magic"):
        abi.parse_ines(b"XES\x1a" + _ines()[4:])
    with pytest.raises(ValueError, match="truncated"):
        abi.parse_ines(_ines()[:-1])
    # Nametable arrangement: flags6 bit 3 four-screen, bit 0 vertical, else horizontal.
    assert abi.parse_ines(_ines(flags6=0x01))["nametable_arrangement"] == 0
    assert abi.parse_ines(_ines(flags6=0x00))["nametable_arrangement"] == 1
    assert abi.parse_ines(_ines(flags6=0x08))["nametable_arrangement"] == 2
    info = abi.parse_ines(synthrom.make_rom(1).rom)
    assert info["prg_rom_size"] == 32768 and info["chr_rom_size"] == 8192 and info["nametable_arrangement"] == 0


def _create(num_envs: int, frameskip: int, rom: bytes, **kw) -> int:
    L = abi.lib()
    cfg = abi.Config()
    L.nesle_config_init(ctypes.byref(cfg))
    cfg.num_envs, cfg.frameskip = num_envs, frameskip
    for k, v in kw.items():
        setattr(cfg, k, v)
    h = ctypes.c_void_p()
    return L.nesle_create(ctypes.byref(cfg), rom, len(rom), ctypes.byref(h))


def test_create_rejects_bad_arguments_before_touching_a_device():
    """num_envs == 0, frameskip == 0, an unknown reward rule, a malformed or
    non-NROM cartridge are invalid arguments (ValueError in the reference)."""
    rom = synthrom.make_rom(1).rom
    L = abi.lib()
    assert _create(0, 4, rom) == abi.EINVAL and "num_envs" in L.nesle_last_error().decode()
    assert _create(abi.MAX_ENVS + 1, 4, rom) == abi.EINVAL and "at most" in L.nesle_last_error().decode()
    assert _create(8, 0, rom) == abi.EINVAL and "frameskip" in L.nesle_last_error().decode()
    assert _create(8, 4, rom, reward_kind=7) == abi.EINVAL
    assert _create(8, 4, b"NES") == abi.EINVAL
    assert _create(8, 4, _ines(flags6=0x10)) == abi.EINVAL and "mapper 0" in L.nesle_last_error().decode()


def test_config_defaults():
    cfg = abi.Config()
    abi.lib().nesle_config_init(ctypes.byref(cfg))
    assert (cfg.frameskip, cfg.max_instructions_per_frame, cfg.reward_kind, cfg.device) == (4, 200000, 0, -1)
    assert (cfg.x_lo, cfg.x_hi, cfg.clip) == (0x86, 0x6D, 15)


def test_null_handles_are_rejected():
    L = abi.lib()
    assert L.nesle_step(None, 0, 0) == abi.EINVAL
    assert L.nesle_reset(None) == abi.EINVAL
    assert L.nesle_num_envs(None) == 0 and L.nesle_device_id(None) == -1


def test_census_field_names_follow_the_header_enum():
    """abi.CENSUS_FIELDS names the census slots in the order of the census
    enum in nesle_amd/csrc/nes_layout.h (k-prefixed CamelCase)."""
    import re

    text = (abi.LIB_PATH.parent / "csrc" / "nes_layout.h").read_text()
    body = text.split("namespace census {", 1)[1].split("kCount", 1)[0]
    body = re.sub(r"//[^\n]*", "", body)
    names = re.findall(r"\bk([A-Z][A-Za-z0-9]*)\b", body)
    snake = [re.sub(r"(?<!^)(?=[A-Z])", "_", n).lower() for n in names]
    assert snake == list(abi.CENSUS_FIELDS)
