"""Native text-artifact readers (``rune_model_load``): malformed files are
rejected with the same messages as the Python readers, which follow the
reference's (rune/mobius/src/mobius.cu:26-151, rune/nep/model.py:284-489).
Parse errors occur before any device work, so these run on the CPU."""

import pytest

from rune_amd import _native as N
from rune_amd.mobius import export as EX
from rune_amd.nep.model import NEP, seeded_nep
from tests.helpers import GOLDEN


def _native_error(path):
    with pytest.raises(ValueError) as info:
        N.NativeModel.load(path)
    return str(info.value)


def _python_error(path):
    with pytest.raises(Exception) as info:
        NEP.from_nep_txt(path)
    return str(info.value)


def test_missing_file_is_reported(tmp_path):
    assert "cannot open" in _native_error(tmp_path / "absent.txt")


@pytest.mark.parametrize("edit, message", [
    (lambda t: t.replace("mobius1 2 Fe C", "mobius1 0", 1), "invalid element count"),
    (lambda t: t.replace("mobius1 2 Fe C", "mobius1 2 Fe Fe", 1), "duplicate elements"),
    (lambda t: t.replace("schema 1", "schema 2", 1), "unsupported native schema"),
    (lambda t: t.replace("\nEND", "\n", 1), "expected 'END' in model file"),
    (lambda t: t + "extra\n", "unexpected data after END"),
    (lambda t: t.rsplit("\n", 3)[0] + "\nEND\n", "missing or nonfinite tensor values"),
    (lambda t: t.replace("ints ", "ints x", 1), "invalid integer metadata count"),
])
def test_malformed_mobius_txt_is_rejected(edit, message, tmp_path):
    text = (GOLDEN / "export_local.mobius.txt").read_text()
    path = tmp_path / "mobius.txt"
    path.write_text(edit(text))
    assert message in _native_error(path)


def _nep_text(tmp_path):
    path = tmp_path / "nep.txt"
    seeded_nep(seed=3).save_nep_txt(path)
    return path.read_text()


@pytest.mark.parametrize("edit", [
    lambda t: t.replace("nep4", "nep5", 1),
    lambda t: t.replace("nep4", "xyz4", 1),
    lambda t: t.replace("ANN 30 0", "ANN 30 1", 1),
    lambda t: t.replace("ANN 30 0", "ANN 300 0", 1),
    lambda t: t.replace("cutoff 6.0 4.0 100 30", "cutoff 6.0 4.0 6.0 4.5 100 30", 1),
    lambda t: t.replace("cutoff 6.0 4.0 100 30", "cutoff 6.0 4.0 100", 1),
    lambda t: t.replace("n_max", "n_mux", 1),
    lambda t: "\n".join(t.split("\n")[:-40]) + "\n",
    lambda t: t.replace("nep4 2 Pb Te", "nep4 3 Pb Te", 1),
])
def test_malformed_nep_txt_matches_python_reader(edit, tmp_path):
    text = _nep_text(tmp_path)
    assert "cutoff 6.0 4.0 100 30" in text and "ANN 30 0" in text
    path = tmp_path / "bad.txt"
    path.write_text(edit(text))
    assert _native_error(path) == _python_error(path)


def test_export_golden_files_exist():
    for kind in ("local", "mp", "eq"):
        assert (GOLDEN / f"export_{kind}.mobius.txt").exists()
    assert EX.read_mobius_txt(GOLDEN / "export_mp.mobius.txt")[0] == ["Fe", "C"]
