"""CPU-side checks of the C-ABI boundary: the library loads and exports every
entry point declared in include/*.h (no compute calls: there is no GPU here)."""
import glob
import os

import tadapt


def test_headers_parse_and_library_exports_every_symbol():
    decl = tadapt.declared()
    assert len(decl) >= 25, sorted(decl)
    L = tadapt.lib()  # raises if any declared symbol is missing
    for name in decl:
        assert hasattr(L, name), name


def test_every_header_declaration_is_bound():
    root = tadapt.ROOT
    for h in glob.glob(os.path.join(root, "include", "*.h")):
        for name in tadapt.parse_header(h):
            assert name in tadapt.declared(), (h, name)


def test_version_and_error_strings():
    assert b"gfx950" in tadapt.lib().ta_version()
    assert isinstance(tadapt.last_error(), str)
