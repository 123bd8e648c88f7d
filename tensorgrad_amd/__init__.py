"""tensorgrad_amd: an MI355X (gfx950) execution backend for tensorgrad's compiled-training path."""
