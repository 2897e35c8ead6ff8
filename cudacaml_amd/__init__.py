"""cudacaml_amd: an MI355X (gfx950) execution backend for CUDACaml's array DSL."""
