"""See the package docstring for the module map."""
